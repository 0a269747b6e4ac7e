// mla_decode.hip -- MI355X (gfx950) split-KV MLA decode: main kernel, LSE combine,
// tile-schedule kernel and the C ABI declared in include/mla_decode_amd.h.
//
// Math (the reference's fp32 oracle, test_mla.py:16-27, generalised to pages,
// per-sequence lengths and causal s_q > 1):
//   S = sm_scale * [q_nope|q_rope] . [kv_nope|kv_rope]^T   (576-d, one shared KV head)
//   O = softmax(S) . kv_nope                                 (512-d, V = first 512 dims of K)
//   lse = log(sum exp S)
//
// Kernel shape.  A workgroup owns one schedule part (a run of 64-token pages, possibly
// spanning several sequences) for one block of R = NW*16*HT query rows, a row being a
// (query token s, head h) pair.  Wave w owns rows [w*16*HT, (w+1)*16*HT) of the block.
// The KV of a part is streamed in 32-token stages (36 KiB: 32 rows x 576 bf16) straight
// from HBM into an LDS ring with global_load_lds_dwordx4 (no VGPR staging); each stage is
// read once from HBM and shared by all waves of the workgroup.
//
// Per stage and wave, everything stays in the MFMA register layouts (16x16x32 bf16/f16):
//   S^T[token, row] = K[token, :] . Q^T[:, row]      A = K from LDS (16-byte reads),
//                                                    B = Q^T, resident in VGPRs
//   P^T = exp2(S^T * sm_scale*log2e - m)             the S^T accumulator layout *is* the
//                                                    B-operand layout of the next product
//   O^T[dim, row] += V^T[dim, token] . P^T[token, row]
//                                                    A = V^T via ds_read_b64_tr_b16 from
//                                                    the same LDS stage (V is never
//                                                    copied or re-read from HBM)
// so the only cross-lane work is the row max / row sum over 4 lane groups.
// The softmax reference max is fixed per segment from its first stage (see ref_tau), so the
// output accumulators are never rescaled; a score far above it triggers an exact two-pass
// redo of the segment.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <math.h>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "mla_decode_amd.h"
#include "mla_sched.h"

namespace mla {

constexpr int kDQK = 576;
constexpr int kDV = 512;
constexpr int kRopeOff = 512;
constexpr int kStageTok = 32;
constexpr int kRowChunks = kDQK / 8;                   // 72 16-byte chunks per token row
constexpr int kRowBytes = kDQK * 2;                    // 1152
constexpr int kStageBytes = kStageTok * kRowBytes;     // 36864
constexpr int kLoadsPerStage = kStageBytes / 1024;     // 36 wave-wide 16-byte loads
constexpr int kPanelBytes = kStageBytes / 2;           // 16 token rows
constexpr int kKSteps = kDQK / 32;                     // 18 k-steps of the QK product
constexpr int kDimTiles = kDV / 16;                    // 32 output dim tiles
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kLog2e = 1.44269504088896340736f;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((__vector_size__(4 * sizeof(short))));
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));
#define LDS_AS __attribute__((address_space(3)))

struct KParams {
  const uint16_t* q_nope;
  const uint16_t* q_rope;
  int64_t q_sb, q_ss, q_sh;
  int64_t qr_sb, qr_ss, qr_sh;
  const uint16_t* kv_nope;
  const uint16_t* kv_rope;
  int64_t kv_sp, kv_st, kv_sb;
  int64_t kr_sp, kr_st, kr_sb;
  const int32_t* block_table;
  int32_t bt_stride;
  int32_t num_blocks;
  // paged: valid columns of the block table; a longer sequence is cut to 64 * bt_width tokens
  // and raises *status (if non-NULL)
  int32_t bt_width;
  int32_t* status;
  const int32_t* seqlens;
  const int32_t* sched;
  const int32_t* splits;
  uint16_t* out;
  int64_t o_sb, o_ss, o_sh;
  float* lse;
  float* ws_lse;    // [slots, rows] log2-domain lse of each split
  float* ws_scale;  // [slots, rows, 4] 2^-e of each 128-dim chunk of a partial row
  uint16_t* ws_o;   // [slots, rows, 512] softmax-normalised partial outputs: fp16 times 2^e
  int32_t part16;   // nonzero: ws_o holds unscaled partials in the input dtype (mla_launch)
  // fp8 latent cache only: kv_nope holds e4m3 codes (strides in bytes) and kv_scale the fp32
  // power-of-two scales, [page][128-dim block][token] with strides ks_sp, ks_sb (floats)
  const float* kv_scale;
  int64_t ks_sp, ks_sb;
  // sparse (top-k) decode only: the keys of sequence b are the pool tokens
  // indices[b * idx_stride + j], j < topk (page id * 64 + row; out of range = no key)
  const int32_t* indices;
  int32_t idx_stride, topk;
  int64_t pool_tokens;
  int32_t batch, s_q, heads, rows, causal, num_parts;
  float scale_log2;  // sm_scale * log2(e)
  // latent and rope halves of one cache tensor (kv_rope = kv_nope + 512, same strides): the
  // wide kernel then reads a row's rope from its latent address + 1024 bytes
  int32_t rope_fused;
};

// ---------------------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------------------

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int DT>
__device__ __forceinline__ f32x4 mfma32(i32x4 a, i32x4 b, f32x4 c) {
  if constexpr (DT == MLA_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// The QK accumulators are kept in VGPRs through inline asm: at one wave per SIMD the compiler
// selects the AGPR form for every MFMA builtin, and the 32-row tile's output accumulator
// (256 registers) already fills the AGPR file.  Operands come straight from LDS / global
// loads; the chain is volatile so no compiler VALU lands between its MFMAs, and
// qk_settle() adds the wait states an MFMA result needs before a VALU may read it.
template <int DT>
__device__ __forceinline__ void mfma_qk_first(f32x4& acc, const i32x4& a, const i32x4& b) {
  if constexpr (DT == MLA_DTYPE_BF16)
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "v"(b));
}
template <int DT>
__device__ __forceinline__ void mfma_qk(f32x4& acc, const i32x4& a, const i32x4& b) {
  if constexpr (DT == MLA_DTYPE_BF16)
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
// 32 wait states after the last QK MFMA: covers the MFMA-result -> VALU-read latency and the
// passes during which the last MFMAs still read their A/B operands.
__device__ __forceinline__ void qk_settle(f32x4& acc) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(acc));
}
__device__ __forceinline__ void qk_touch(f32x4& acc) { asm volatile("" : "+v"(acc)); }
// 12 wait states for the QK accumulators when at least eight other MFMAs have issued since the
// last QK MFMA (20 in all, the most any MFMA result needs before a VALU read).
template <int HT>
__device__ __forceinline__ void qk_settle_after_mfmas(f32x4 (&acc)[HT][2]) {
  if constexpr (HT == 2)
    asm volatile("s_nop 7\n\ts_nop 3" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]));
  else
    asm volatile("s_nop 7\n\ts_nop 3" : "+v"(acc[0][0]), "+v"(acc[0][1]));
}

// 32 wait states during which the MFMA source operands passed in stay untouched.
template <int HT>
__device__ __forceinline__ void operand_guard(i32x4 (&pb)[HT], i32x4& va) {
  if constexpr (HT == 2)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(pb[0]), "+v"(pb[1]), "+v"(va));
  else
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(pb[0]), "+v"(va));
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two floats rounded to nearest even and packed low-first: one v_cvt_pk_{bf16,f16}_f32.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2 v = {a, b};
  if constexpr (DT == MLA_DTYPE_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// Split partials in the decode workspace are fp16 with one power-of-two scale 2^e per (row,
// 128-dim chunk), e chosen from the chunk's amax so that it lands in [2^14, 2^15): every value
// is then held to 2^-11 of the chunk's amax, half the bytes of fp32 partials (bf16 partials
// would move merged outputs in [2, 4) past the 1e-2 bar).  The workspace keeps 2^-e.
__device__ __forceinline__ int part_exp(float amax) {
  const int e = 15 - __builtin_amdgcn_frexp_expf(amax);  // amax = m * 2^E, m in [0.5, 1); 0 -> E = 0
  return e < 127 ? e : 127;                               // amax < 2^-112: still below 2^15
}
__device__ __forceinline__ float exp2i(int e) {  // 2^e for e in [-126, 127]
  return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
}
__device__ __forceinline__ float amax4(const f32x4 v) {
  return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
}

// acc + the sum of the eight 16-bit values packed in w (one v_dot2c_f32_{bf16,f16} per pair,
// fp32 accumulation).  The softmax row sums are taken over the P values as rounded for the PV
// product, so the weights applied to V sum to exactly the denominator.
template <int DT>
__device__ __forceinline__ float packed_sum(const i32x4 w, float acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t x = (uint32_t)w[j];  // element copied out before the bit cast
    if constexpr (DT == MLA_DTYPE_BF16)
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), bf16x2{(__bf16)1.f, (__bf16)1.f}, acc,
                                            false);
    else
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), f16x2{(_Float16)1, (_Float16)1}, acc, false);
  }
  return acc;
}

// max of three floats in one v_max3_f32 (fmaxf would first canonicalise each operand for
// signalling-NaN semantics; scores here are finite or -inf)
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

template <int DT>
__device__ __forceinline__ float to_f32(uint16_t v) {
  if constexpr (DT == MLA_DTYPE_BF16) {
    return __uint_as_float((uint32_t)v << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, v);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One wave-wide 16-byte-per-lane HBM -> LDS copy (global_load_lds_dwordx4, SGPR-base form):
// lane l reads base + voff_l and its 16 bytes land at LDS byte lds_addr + 16*l.  Issued as
// inline asm on purpose: the compiler then does not track it as an LDS store, so it adds no
// conservative vmcnt(0) waits before the LDS reads of *other* stages; completion is awaited
// explicitly (wait_stage) before a barrier.  M0 (the LDS base of the copy) is written without
// a save/restore: M0 is a reserved register, which clang does not preserve for a clobber, and
// nothing else in these kernels reads it (no LDS-DMA builtins, message sends or relative
// register moves; the generated code has no M0 reader besides these copies).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds_addr) {
  // base and lds_addr are uniform; readfirstlane makes that visible to the register allocator.
  // The builtin returns a signed int: each half goes through uint32_t before widening, or a
  // low word with bit 31 set would sign-extend into the high word.
  const uint64_t b64 = (uint64_t)(uintptr_t)base;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b64);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b64 >> 32));
  const uint64_t sbase = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %0, %1 nt"
      :
      : "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
      : "memory", "m0");
}
// The same copy with the LDS destination given as an SGPR plus an immediate (one SALU op,
// written straight into M0) and the global address stepped by the instruction's immediate
// offset GOFF: the wide kernel's stage loads.  The immediate offset moves the LDS destination
// too (LDS address = M0 + offset + 16 * lane), so M0 takes LDS_OFF - GOFF and the copy lands
// at lds_base + LDS_OFF; a load then costs one scalar instruction and no vector one.  Without
// the non-temporal hint: workgroups that stream the same pages (the head blocks of a part,
// neighbouring splits) find them in L2 (measured: 12% fewer fetched bytes at 256 rows, 9%
// faster at 64 rows).
template <int LDS_OFF, int GOFF = 0, bool NT = false>
__device__ __forceinline__ void dma16_m0(uint64_t sbase, uint32_t voff, uint32_t lds_base) {
  static_assert(GOFF >= 0 && GOFF < 4096 && LDS_OFF - GOFF > -65536, "immediate offset range");
  if constexpr (NT) {
    asm volatile(
        "s_add_u32 m0, %2, %3\n\t"
        "global_load_lds_dwordx4 %0, %1 offset:%4 nt"
        :
        : "v"(voff), "s"(sbase), "s"(lds_base), "i"(LDS_OFF - GOFF), "i"(GOFF)
        : "memory", "m0", "scc");
  } else {
    asm volatile(
        "s_add_u32 m0, %2, %3\n\t"
        "global_load_lds_dwordx4 %0, %1 offset:%4"
        :
        : "v"(voff), "s"(sbase), "s"(lds_base), "i"(LDS_OFF - GOFF), "i"(GOFF)
        : "memory", "m0", "scc");
  }
}
// The same copy from a per-lane 64-bit address (the sparse path: every token row has its own
// page).
__device__ __forceinline__ void dma16_lane(const void* addr, uint32_t lds_addr) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %0, off nt"
      :
      : "v"(addr), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
      : "memory", "m0");
}
// 4 bytes per lane from a per-lane address, to LDS at lds_addr + 4 * lane (sparse fp8 scales).
__device__ __forceinline__ void dma4_lane(const void* addr, uint32_t lds_addr) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dword %0, off nt"
      :
      : "v"(addr), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
      : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier for LDS hand-off only.  Each wave has already waited for its own DMA
// copies (vmcnt) and consumed its own LDS reads, so no memory-model fence is needed (the
// fence __syncthreads() implies would wait for every in-flight stage load); the empty asm
// statements keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Lane l's value and lane (l ^ 16)'s, or (l ^ 32)'s, as the two halves of one v_permlane16_swap /
// v_permlane32_swap of v with itself (lanes 0..31 receive the other row's value in the second
// half, lanes 32..63 in the first; either way the pair is {v[l], v[l ^ d]}).  No LDS and no lane
// id: __shfl_xor goes through ds_bpermute with an address formed from the lane id, which the
// compiler computes once per kernel and, under register pressure, spills; the reload then waits
// (vmcnt is in order) for every stage load in flight.
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_max_g(float v) {
  // max over the 4 lane groups (lanes l, l^16, l^32, l^48) that hold one row
  return xor32_max(xor16_max(v));
}
__device__ __forceinline__ float wave_sum_g(float v) {
  return xor32_sum(xor16_sum(v));
}
// -inf, materialised where it is called (a constant would be hoisted out of a rarely taken branch)
__device__ __forceinline__ float neg_inf_here() {
  float v;
  asm volatile("v_mov_b32 %0, 0xff800000" : "=v"(v));
  return v;
}
// The lane id, computed afresh where it is called (two VALU ops the compiler cannot hoist):
// lane-dependent addresses formed from it stay inside the segment or pass that uses them
// instead of being computed once per kernel and spilled.
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// ---------------------------------------------------------------------------------------
// stage loads: HBM -> LDS, 36 wave-wide 16-byte loads per 32-token stage
// ---------------------------------------------------------------------------------------
// LDS layout of a stage (32 token rows of 72 16-byte chunks): 36 blocks of 1 KiB.  Block
// q*9 + s (q = 0..3) holds token rows 8q .. 8q+7 (row group q: panel q/2, half q%2) and
// chunks 8s .. 8s+7 (s = 8: the rope dims); inside a block, chunk 8s + c8 of row r sits at
// 16-byte slot 8*(r%8) + (c8 ^ swz(r % 16)), with
//   swz(r) = 2*((r/2) % 4) + r/8.
// One wave-wide global_load_lds_dwordx4 fills one block: lane l fetches row 8q + l/8, chunk
// 8s + ((l%8) ^ swz), so the eight lanes of a row cover one whole 128-byte line and every
// load reads eight full lines (which the non-temporal policy streams at ~15% more bandwidth
// than half-line accesses; half lines under that policy are fetched twice).  The swizzle
// keeps the fragment reads conflict-free: the sixteen rows of one chunk (QK A operand) and
// the 4-row x 2-chunk V^T blocks of one transposed read spread over all 64 banks.
__device__ __forceinline__ int stage_swz(int r) { return (((r >> 1) & 3) << 1) | ((r >> 3) & 1); }

template <int NL>
__device__ __forceinline__ void issue_stage(uint8_t LDS_AS* slot, const uint16_t* nope_base,
                                            const uint16_t* rope_base, int kv_st, int kr_st,
                                            int last_row, int wave, int lane) {
  // NL = 4: wave w loads row group w (9 blocks); NL = 1: the wave loads all 36 blocks.
  static_assert(NL == 1 || NL == 4, "stage loads are split over one or four waves");
#pragma unroll
  for (int qi = 0; qi < 4 / NL; ++qi) {
    const int q = NL == 1 ? qi : wave;  // uniform
    // Rows past the sequence end re-read its last row: in bounds, finite, masked later.
    int row = 8 * q + (lane >> 3);
    row = row < last_row ? row : last_row;
    const uint32_t cl = (uint32_t)(((lane & 7) ^ stage_swz(((q & 1) << 3) | (lane >> 3))) << 4);
    const uint32_t on = (uint32_t)(row * kv_st) * 2 + cl;
    const uint32_t orp = (uint32_t)(row * kr_st) * 2 + cl;
    uint8_t LDS_AS* dst = slot + q * 9 * 1024;
#pragma unroll
    for (int sg = 0; sg < 8; ++sg)
      dma16((const char*)nope_base + 128 * sg, on, (uint32_t)(uintptr_t)(dst + sg * 1024));
    dma16(rope_base, orp, (uint32_t)(uintptr_t)(dst + 8 * 1024));
  }
}

// Sparse (top-k) decode: the same stage layout, each token row fetched from its own pool token
// (idx_stage[r] = page * 64 + row); rows past the list's end re-read its last row, and an index
// outside the pool reads pool token 0 (both are masked by the caller).
constexpr int kSparseMaxTopk = 2048;
template <int NL>
__device__ __forceinline__ void issue_stage_sparse(uint8_t LDS_AS* slot, const uint16_t* nope_pool,
                                                   const uint16_t* rope_pool,
                                                   const int32_t LDS_AS* idx_stage, int valid_rows,
                                                   int64_t kv_sp, int64_t kv_st, int64_t kr_sp,
                                                   int64_t kr_st, int64_t pool_tokens, int wave,
                                                   int lane) {
  static_assert(NL == 1 || NL == 4, "stage loads are split over one or four waves");
#pragma unroll
  for (int qi = 0; qi < 4 / NL; ++qi) {
    const int q = NL == 1 ? qi : wave;  // uniform
    const int r = 8 * q + (lane >> 3);
    const int t = r < valid_rows ? r : valid_rows - 1;
    int64_t idx = idx_stage[t];
    if (idx < 0 || idx >= pool_tokens) idx = 0;
    const int64_t pg = idx >> 6, rw = idx & 63;
    const uint32_t cl = (uint32_t)(((lane & 7) ^ stage_swz(((q & 1) << 3) | (lane >> 3))) << 4);
    const char* nrow = (const char*)(nope_pool + pg * kv_sp + rw * kv_st) + cl;
    const char* rrow = (const char*)(rope_pool + pg * kr_sp + rw * kr_st) + cl;
    uint8_t LDS_AS* dst = slot + q * 9 * 1024;
#pragma unroll
    for (int sg = 0; sg < 8; ++sg) dma16_lane(nrow + 128 * sg, (uint32_t)(uintptr_t)(dst + sg * 1024));
    dma16_lane(rrow, (uint32_t)(uintptr_t)(dst + 8 * 1024));
  }
}

template <int PER, int NSTAGE>
__device__ __forceinline__ void wait_stage(int after) {
  // Wait until this wave's loads of the oldest outstanding stage have landed (PER loads per
  // stage and wave), with `after` younger stages allowed to stay in flight.
  constexpr int per = PER;
  if constexpr (NSTAGE >= 4) {
    if (after >= 2) { wait_vmcnt<(2 * per < 64 ? 2 * per : 0)>(); return; }
  }
  if constexpr (NSTAGE >= 3) {
    if (after >= 1) { wait_vmcnt<(per < 64 ? per : 0)>(); return; }
  }
  wait_vmcnt<0>();
}

__device__ __forceinline__ i32x4 lds_tr_pair(const uint8_t LDS_AS* p) {
  // Two transposed 4x16 reads, one per 16-row panel: lane (g, i) gets V^T[i][4g..4g+3] and
  // V^T[i][16+4g..16+4g+3] of the 16-column block its lane group addressed.
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 LDS_AS*)p);
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 LDS_AS*)(p + kPanelBytes));
  const i32x2 lo2 = __builtin_bit_cast(i32x2, lo);
  const i32x2 hi2 = __builtin_bit_cast(i32x2, hi);
  return i32x4{lo2.x, lo2.y, hi2.x, hi2.y};
}

// ---------------------------------------------------------------------------------------
// fp8 latent cache: stage layout, loads and fragment conversion
// ---------------------------------------------------------------------------------------
// A stage of the fp8 cache (32 token rows, 24 KiB of LDS):
//   - latent codes: block q*4 + s (q = row group 0..3: rows 8q .. 8q+7; s = 128-byte segment
//     0..3 of the 512-byte row) holds 16-byte chunk c16 of row r at slot
//     8*(r%8) + (c16 ^ swz8(r)),  swz8(r) = (r%8)/2 + 4*((r/8 ^ r/16) & 1);
//   - rope (bf16): 16 KiB + block q, 16-byte chunk c (8 dims) of row r at slot
//     8*(r%8) + (c ^ swzr(r)),  swzr(r) = (r%8)/2 + 4*((r/8) & 1);
//   - scales: 20 KiB + 1 KiB * blk, the fp32 scale of 128-dim block blk of token t at byte 4t.
// Every latent and rope load reads eight whole 128-byte lines.  The swizzles keep the QK
// fragment reads (8 bytes of 16 rows x 2 lane groups, or 16 bytes of 16 rows) and the
// transposed V^T reads (8 rows x 16 bytes per lane-group pair) free of bank conflicts.
constexpr int kStageBytes8 = 24 * 1024;
constexpr int kLoadsPerStage8 = 24;
constexpr int kRopeOff8 = 16 * 1024;
constexpr int kScaleOff8 = 20 * 1024;
__device__ __forceinline__ int swz8(int r) { return ((r & 7) >> 1) | ((((r >> 3) ^ (r >> 4)) & 1) << 2); }
__device__ __forceinline__ int swzr(int r) { return ((r & 7) >> 1) | (((r >> 3) & 1) << 2); }

template <int NL>
__device__ __forceinline__ void issue_stage8(uint8_t LDS_AS* slot, const uint8_t* lat_base,
                                             const uint16_t* rope_base, const float* scale_base,
                                             int lat_st, int rope_st, int64_t scale_sb,
                                             int last_row, int wave, int lane) {
  // NL = 4: wave w loads row group w's 4 latent blocks and rope block, and the scales of
  // 128-dim block w; NL = 1: the wave loads all 24 blocks.
  static_assert(NL == 1 || NL == 4, "stage loads are split over one or four waves");
#pragma unroll
  for (int qi = 0; qi < 4 / NL; ++qi) {
    const int q = NL == 1 ? qi : wave;  // uniform
    const int r = 8 * q + (lane >> 3);  // LDS row; rows past the sequence end re-read its last row
    const int row = r < last_row ? r : last_row;
    const uint32_t on = (uint32_t)(row * lat_st) + (uint32_t)(((lane & 7) ^ swz8(r)) << 4);
    const uint32_t orp = (uint32_t)(row * rope_st) * 2 + (uint32_t)(((lane & 7) ^ swzr(r)) << 4);
#pragma unroll
    for (int sg = 0; sg < 4; ++sg)
      dma16(lat_base + 128 * sg, on, (uint32_t)(uintptr_t)(slot + (q * 4 + sg) * 1024));
    dma16(rope_base, orp, (uint32_t)(uintptr_t)(slot + kRopeOff8 + q * 1024));
    // 32 token scales of block q: lanes 0..7 fetch 16 bytes each, the others repeat them
    dma16(scale_base + q * scale_sb, (uint32_t)((lane & 7) << 4),
          (uint32_t)(uintptr_t)(slot + kScaleOff8 + q * 1024));
  }
}

// Sparse decode over the fp8 cache: the same stage layout, each token row gathered from its own
// pool token (idx_stage[r] = page * 64 + row; rows past the list's end re-read its last row, an
// id outside the pool reads pool token 0, both masked by the caller).  The scales of the stage's
// 32 tokens for 128-dim block q are 32 separate floats, gathered by one 4-byte load per lane
// (lanes 32..63 repeat lanes 0..31 into the unused upper part of the block's scale slot).
// NL = 4: wave w loads row group w and the scales of block w; NL = 1: everything.
template <int NL>
__device__ __forceinline__ void issue_stage8_sparse(uint8_t LDS_AS* slot, const uint8_t* lat_pool,
                                                    const uint16_t* rope_pool, const float* scale_pool,
                                                    const int32_t LDS_AS* idx_stage, int valid_rows,
                                                    int64_t lat_sp, int64_t lat_st, int64_t kr_sp,
                                                    int64_t kr_st, int64_t ks_sp, int64_t ks_sb,
                                                    int64_t pool_tokens, int wave, int lane) {
  static_assert(NL == 1 || NL == 4, "stage loads are split over one or four waves");
  auto token = [&](int r) {
    const int t = r < valid_rows ? r : valid_rows - 1;
    int64_t idx = idx_stage[t];
    return (idx < 0 || idx >= pool_tokens) ? (int64_t)0 : idx;
  };
#pragma unroll
  for (int qi = 0; qi < 4 / NL; ++qi) {
    const int q = NL == 1 ? qi : wave;  // uniform
    const int r = 8 * q + (lane >> 3);
    const int64_t idx = token(r);
    const int64_t pg = idx >> 6, rw = idx & 63;
    const uint8_t* lrow = lat_pool + pg * lat_sp + rw * lat_st + (((lane & 7) ^ swz8(r)) << 4);
    const char* rrow = (const char*)(rope_pool + pg * kr_sp + rw * kr_st) + (((lane & 7) ^ swzr(r)) << 4);
#pragma unroll
    for (int sg = 0; sg < 4; ++sg) dma16_lane(lrow + 128 * sg, (uint32_t)(uintptr_t)(slot + (q * 4 + sg) * 1024));
    dma16_lane(rrow, (uint32_t)(uintptr_t)(slot + kRopeOff8 + q * 1024));
    const int64_t sidx = token(lane & 31);
    const float* sc = scale_pool + (sidx >> 6) * ks_sp + q * ks_sb + (sidx & 63);
    dma4_lane(sc, (uint32_t)(uintptr_t)(slot + kScaleOff8 + q * 1024));
  }
}

// Two OCP e4m3 codes (bytes 2*hi, 2*hi+1 of w) to two bf16 values times 2^exponent(scale).
template <bool HI>
__device__ __forceinline__ int cvt_fp8x2(int w, float scale) {
  return __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, scale, HI));
}
__device__ __forceinline__ i32x4 cvt_fp8x8(i32x2 raw, float scale) {
  const int x = raw.x, y = raw.y;  // elements copied out before use (see the bit_cast note)
  return i32x4{cvt_fp8x2<false>(x, scale), cvt_fp8x2<true>(x, scale), cvt_fp8x2<false>(y, scale),
               cvt_fp8x2<true>(y, scale)};
}

// ---------------------------------------------------------------------------------------
// main split-KV kernel
// ---------------------------------------------------------------------------------------
// Softmax reference.  A segment (the run of pages of one sequence a part owns) fixes its
// reference row max m from the scores of its first stage; every later P = 2^(s*c - m) then
// stays below 2^tau, which is finite in the 16-bit type P is rounded to and leaves fp32
// sums far from overflow, so the output accumulators are never rescaled.  Should a later
// score exceed m + tau, the whole workgroup abandons the pass and redoes the segment in two
// passes: one that only finds the exact row max, one that accumulates against it.
template <int DT>
constexpr float ref_tau() {
  return DT == MLA_DTYPE_BF16 ? 64.f : 15.f;
}

enum PassMode { kPassFirstStageRef = 0, kPassRowMax = 1, kPassFixedRef = 2 };

__device__ __forceinline__ void wait_lgkm0() {
  // lgkmcnt(0), vmcnt / expcnt left at their maxima
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

// Sequence b's length as the kernels use it: negative lengths read as 0, and a paged sequence
// longer than its block-table row (64 * bt_width tokens) is cut there, so no column past the
// table's width is read; that raises the caller's status word (every lane stores the same 1).
__device__ __forceinline__ int bound_seq_len(const KParams& p, int L, bool paged) {
  L = L > 0 ? L : 0;
  if (paged) {
    const int cap = p.bt_width * kPageTokens;  // bt_width <= 2^24, checked by the host
    if (L > cap) {  // uniform
      L = cap;
      if (p.status != nullptr) *p.status = 1;
    }
  }
  return L;
}
__device__ __forceinline__ int seq_len_bounded(const KParams& p, int b, bool paged) {
  return bound_seq_len(p, p.seqlens[b], paged);
}

// Waves per SIMD a variant is compiled for: four waves of one 16-row tile each with at most
// a 2-stage ring fit 256 registers, so two workgroups share a CU; everything else takes the
// whole register file (one wave per SIMD).
constexpr int waves_per_simd(int nw, int ht, int nstage, bool ws) {
  return (!ws && ht == 1 && nw == 4 && nstage <= 2) ? 2 : 1;
}

// Two ways to use the NW waves of a workgroup:
//  - WS = false: each wave owns its own 16*HT rows (R = NW*16*HT rows per workgroup) and all
//    waves share one NSTAGE ring: every stage is loaded once, by all waves together, and
//    consumed by all of them (a barrier per stage);
//  - WS = true ("wave split", NSTAGE = 1): the waves share one 16*HT-row tile and take turns
//    over the segment's stages (wave w takes stages w, w + NW, ...), each loading its own
//    stages into its own one-stage slot with no barrier between waves; their accumulators are
//    merged through LDS at the end of the segment, so the workgroup leaves one partial where
//    NW single-wave workgroups would leave NW.
// KV8: the latent cache holds OCP e4m3 codes with power-of-two scales per token and 128-dim
// block (bf16 queries and rope); K fragments are converted to bf16 with their scale on the way
// from LDS to the MFMA, V^T fragments without it, and the scales of V are folded into P^T.
// SPARSE: the keys of a sequence are the top-k pool tokens its index list names (s_q = 1).
// (HIP's second launch bound is the minimum number of waves per SIMD, amdgpu_waves_per_eu.)
// The schedule comes as a scalar argument of its own besides p.sched: the build preloads scalar
// kernel arguments into SGPRs (-amdgpu-kernarg-preload-count), so the first record load does
// not wait for the argument segment (a struct argument is never preloaded).
template <int DT, int NW, int HT, int NSTAGE, bool WS, bool KV8, bool SPARSE = false>
__global__ __launch_bounds__(NW * 64, waves_per_simd(NW, HT, NSTAGE, WS))
void mla_splitkv_kernel(const int32_t* __restrict__ sched, KParams p) {
  static_assert(NW == 1 || NW == 4, "one or four waves per workgroup");
  static_assert(!WS || NSTAGE == 1, "wave-split workgroups give each wave a one-stage slot");
  static_assert(!KV8 || DT == MLA_DTYPE_BF16, "the fp8 cache is read with bf16 queries");
  constexpr int kSB = KV8 ? kStageBytes8 : kStageBytes;      // bytes of one stage in LDS
  constexpr int kLPS = KV8 ? kLoadsPerStage8 : kLoadsPerStage;  // wave-wide loads per stage
  constexpr int NL = WS ? 1 : NW;  // waves sharing the loads of one stage
  constexpr int LEAD = NSTAGE - 1;
  static_assert((NSTAGE - 1) * (kLPS / NL) < 64, "outstanding stage loads exceed vmcnt");
  static_assert(kLPS % NL == 0, "loads per stage must split evenly");
  constexpr int R = WS ? 16 * HT : NW * 16 * HT;
  constexpr int DK = 4;  // LDS prefetch depth of the QK A fragments
  constexpr int DV = HT == 2 ? 2 : 4;  // LDS prefetch depth of the PV A fragments
  constexpr float kTau = ref_tau<DT>();
  constexpr int kSlots = WS ? NW : NSTAGE;
  constexpr int kMergePitch = kDV * 4 + 16;  // wave-split merge: fp32 rows of 512, padded
  constexpr int kMergeBytes = WS ? NW * 16 * kMergePitch : 0;
  constexpr int kSmem = kSlots * kSB > kMergeBytes ? kSlots * kSB : kMergeBytes;
  // fp8 with four loading waves: each stage is dequantised once, a row group per wave, into a
  // bf16 stage buffer, and the bf16 fragment path reads it (kDeq); the one-wave layouts convert
  // every fragment on its way to the MFMA instead (kInl8).
  constexpr bool kDeq = KV8 && NL == 4;
  constexpr bool kInl8 = KV8 && !kDeq;
  // wave split, dense 16-bit cache: a wave refills its slot with its next own stage while it
  // still computes the current one (rope blocks after QK, each 64-dim latent segment once PV
  // has read it), instead of in one burst after PV
  constexpr bool kProg = WS && !(SPARSE && KV8);
  __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[kSmem + (kDeq ? kStageBytes : 0)];
  // wave-split merge words: (row max, row sum of rounded P, row sum of fp32 P) per wave and row
  __shared__ float merge_sh[WS ? NW : 1][3][16];
  // sparse: the pool-token indices of the current segment
  __shared__ int32_t idx_sh[SPARSE ? kSparseMaxTopk : 1];
  // "score above reference" words, one per stage modulo 4.  A wave whose stage-k scores exceed
  // the reference stores 1 into over_sh[k % 4] (a wave-uniform branch, all lanes storing the
  // same value); every wave reads the word after the next barrier; wave 0 clears it two
  // stages later, once every wave has read it, and two barriers separate that clear from the
  // word's next use.
  __shared__ int over_sh[4];
  uint8_t LDS_AS* smem = (uint8_t LDS_AS*)smem_raw;

  const int part = blockIdx.x;
  const int hb = blockIdx.y;
  // wave index made explicitly uniform, so per-wave choices compile to scalar code
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;   // lane group (MFMA k quarter / output row quarter)
  const int li = lane & 15;  // lane within group
  const int row0 = hb * R + (WS ? 0 : wave * 16 * HT);
  // this wave's stage ring, and the first stage / stride of its turn over a segment
  uint8_t LDS_AS* const ring = smem + (WS ? wave * kSB : 0);
  uint8_t LDS_AS* const deq = smem + kSmem;  // kDeq: the bf16 stage
  const int k0 = WS ? wave : 0;
  constexpr int kStep = WS ? NW : 1;

  const int32_t* rec = sched + part * kSchedWords;
  int b = rec[0];
  int page = rec[1];
  const int end_b = rec[2];
  const int end_page = rec[3];
  int split = rec[4];

  // Per-lane LDS byte offsets that do not depend on the stage (block layout above).
  // QK A operand, fragment (kk, tt): token row 16*tt + li of chunk sigma(kk, g), where
  //   sigma(kk, g) = 8*(kk/2) + 2*g + kk%2,
  // i.e. block (2tt + li/8)*9 + kk/2, chunk-in-block 2g + kk%2: one lane offset per parity of
  // kk, the rest (tt, kk/2) an immediate.  The query fragments use the same sigma.
  const int k_lane0 = (li >> 3) * 9216 + ((((li & 7) << 3) + ((2 * g) ^ stage_swz(li))) << 4);
  const int k_lane1 = (li >> 3) * 9216 + ((((li & 7) << 3) + ((2 * g + 1) ^ stage_swz(li))) << 4);
  // V^T A operand, dim tile dt = 4s + d4: the lane addresses token row rv = 4g + li/4 (and the
  // same row of the second panel), bytes 32*dt + 8*(li%4), i.e. chunk 8s + 2*d4 + (li%4)/2 in
  // block (rv/8)*9 + s.  The chunk's swizzle only flips bits 5-6 of the address with d4, so the
  // address of tile dt is (v_lane ^ 32*d4) + 1024*s over a 1 KiB-aligned stage base.
  const int rv = 4 * g + (li >> 2);
  const int v_lane = (rv >> 3) * 9216 + ((rv & 7) << 7) + (((li >> 1) & 1) ^ stage_swz(rv)) * 16 +
                     ((li & 1) << 3);
  // fp8 layout (KV8).  QK: latent fragment (kk < 16, tt) = token row 16tt + li, dims
  // 32kk + 8g .. +7 (8 bytes): block (2tt + li/8)*4 + kk/4, chunk 2(kk%4) + g/2, half g%2; with
  // swz8(16tt + li) = swz8(li) ^ 4tt the address is (kb8 ^ 32(kk%4) ^ 64tt) + 8192tt +
  // 1024(kk/4).  Rope fragment kk = 16 + j: chunk 4j + g of rope block 2tt + li/8, address
  // (kr8 ^ 64j) + 2048tt.  PV: lane li of group g addresses token t8 = (li/2 < 4 ? 4g + li/2 :
  // 12 + 4g + li/2), byte half li%2 of chunk dt%8 in block (t8/8)*4 + dt/8; ds_read_b64_tr_b8
  // hands lane li the 8 tokens its group addressed at dim 16dt + li, i.e. the V^T A operand
  // whose k order (tokens 4g..4g+3, 16+4g..16+4g+3) is that of P^T.  Address of tile dt:
  // (v8_lane ^ 16(dt%8)) + 1024(dt/8).
  const int kb8 = (li >> 3) * 4096 + ((((li & 7) << 3) + ((g >> 1) ^ swz8(li))) << 4) + ((g & 1) << 3);
  const int kr8 = kRopeOff8 + (li >> 3) * 1024 + ((((li & 7) << 3) + (g ^ swzr(li))) << 4);
  const int t8 = (li >> 1) < 4 ? 4 * g + (li >> 1) : 12 + 4 * g + (li >> 1);
  const int v8_lane = (t8 >> 3) * 4096 + ((((t8 & 7) << 3) + swz8(t8)) << 4) + ((li & 1) << 3);

  const int kv_st = (int)p.kv_st, kr_st = (int)p.kr_st;
  const bool paged = p.block_table != nullptr;

#pragma unroll 1
  for (; b < p.batch; ++b, page = 0, split = 0) {
    if (!(b < end_b || (b == end_b && page < end_page))) break;
    // Segment prologue: the first 64 page ids, the query fragments and the length are requested
    // back to back, in that order, so the segment starts after two memory round trips (these
    // loads, then its first stage) instead of one per dependent load.
    int pbase = 0, bt_lane = 0;
    // lane i holds the page id of page (pbase + i), clamped into the pool; the columns read stop
    // at the table's width, not at the sequence's last page, so the load does not wait for the
    // length (only the ids of the sequence's own pages are ever used)
    auto request_page_ids = [&](int first) __attribute__((always_inline)) {
      pbase = first;
      if (paged && !SPARSE) {
        const int last = p.bt_width - 1;
        const int pi = pbase + lane < last ? pbase + lane : last;
        bt_lane = p.block_table[(int64_t)b * p.bt_stride + pi];
      }
    };
    auto finish_page_ids = [&]() __attribute__((always_inline)) {
      if (paged && !SPARSE) {
        const int v = bt_lane;
        bt_lane = v < 0 ? 0 : (v >= p.num_blocks ? p.num_blocks - 1 : v);
      }
    };
    auto load_page_ids = [&](int first) __attribute__((always_inline)) {
      request_page_ids(first);
      finish_page_ids();
    };
    request_page_ids(page);
    // The sequence's workspace slots, for the epilogue.  The index carries an opaque zero, so
    // the compiler treats the values as per-lane: it neither moves them into SGPRs (waiting for
    // them) here nor loads them in the epilogue; they are made uniform where they are used.
    const int zero_v = fresh_lane() >> 6;
    const int slot_lo_v = p.splits[b + zero_v];
    const int slot_hi_v = p.splits[b + 1 + zero_v];

    // ---- query fragments (B operand of S^T = K Q^T), resident for the segment.  Rows
    // past the end re-load the last row; their results are never written.
    i32x4 qf[HT][kKSteps];
    int qtok[HT];  // query token of each row tile's row
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      int row = row0 + 16 * ht + li;
      row = row < p.rows ? row : p.rows - 1;
      const int s = row / p.heads;
      const int h = row - s * p.heads;
      qtok[ht] = s;
      const uint16_t* qn = p.q_nope + (b * p.q_sb + s * p.q_ss + h * p.q_sh) + 16 * g;
      const uint16_t* qr = p.q_rope + (b * p.qr_sb + s * p.qr_ss + h * p.qr_sh) + 16 * g;
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        if constexpr (kInl8) {
          // dims 32kk + 8g (the fp8 fragments' natural order)
          const int d = 32 * kk - 8 * g;  // qn / qr already point 16g past the row start
          qf[ht][kk] = *(const i32x4*)(kk < 16 ? qn + d : qr + (d - kRopeOff));
        } else {
          // dims 8*sigma(kk, g) = 64*(kk/2) + 16*g + 8*(kk%2)
          const int d = 64 * (kk >> 1) + 8 * (kk & 1);
          qf[ht][kk] = *(const i32x4*)(d < kRopeOff ? qn + d : qr + (d - kRopeOff));
        }
      }
    }
    // the length and the sequence's workspace slots (loaded here so that the epilogue does not
    // wait on them) last: awaiting them also awaits everything above (vmcnt is in order), which
    // is in flight by then
    const int L = SPARSE ? p.topk : bound_seq_len(p, p.seqlens[b], paged);
    finish_page_ids();
    const int np = pages_of(L);
    const int stop = (b == end_b) ? end_page : np;
    const int st_begin = 2 * page;
    const int st_end_seq = (L + kStageTok - 1) / kStageTok;
    const int st_end = (2 * stop < st_end_seq) ? 2 * stop : st_end_seq;
    const int nst = st_end > st_begin ? st_end - st_begin : 0;
    int lim[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) lim[ht] = L - (p.causal ? (p.s_q - 1 - qtok[ht]) : 0);
    const int lmin = L - (p.causal ? p.s_q - 1 : 0);  // every row sees tokens < lmin
    if constexpr (SPARSE) {
      // the segment's index list into LDS (every wave of the workgroup runs this segment; the
      // previous segment's readers are past its final barrier)
      const int tok0 = st_begin * kStageTok;
      int ntok = L - tok0;
      ntok = ntok < nst * kStageTok ? ntok : nst * kStageTok;
      for (int i = threadIdx.x; i < ntok; i += NW * 64) idx_sh[i] = p.indices[(int64_t)b * p.idx_stride + tok0 + i];
      wait_lgkm0();
      lds_barrier();
    }

    f32x4 o[kDimTiles][HT];
    // row sums: l_part of P as rounded for the PV product (normalises the output), l_exact of
    // the fp32 P (gives the lse)
    float m_ref[HT], l_part[HT], l_exact[HT];

    auto issue = [&](int k) __attribute__((always_inline)) {
      const int st = st_begin + k;
      if constexpr (SPARSE && KV8) {
        const int left = L - st * kStageTok;
        issue_stage8_sparse<NL>(ring + (k % NSTAGE) * kSB, (const uint8_t*)p.kv_nope, p.kv_rope, p.kv_scale,
                                (const int32_t LDS_AS*)idx_sh + k * kStageTok,
                                left < kStageTok ? left : kStageTok, p.kv_sp, p.kv_st, p.kr_sp, p.kr_st,
                                p.ks_sp, p.ks_sb, p.pool_tokens, NL == 1 ? 0 : wave, lane);
        return;
      } else if constexpr (SPARSE) {
        const int left = L - st * kStageTok;
        issue_stage_sparse<NL>(ring + (k % NSTAGE) * kSB, p.kv_nope, p.kv_rope,
                               (const int32_t LDS_AS*)idx_sh + k * kStageTok,
                               left < kStageTok ? left : kStageTok, p.kv_sp, p.kv_st, p.kr_sp, p.kr_st,
                               p.pool_tokens, NL == 1 ? 0 : wave, lane);
        return;
      }
      if constexpr (KV8) {  // paged only (checked by the host)
        const int pidx = st >> 1;
        if (pidx - pbase >= 64) load_page_ids(pidx);  // uniform
        const int pg = __builtin_amdgcn_readlane(bt_lane, pidx - pbase);
        const int tok = (st & 1) * kStageTok;
        const uint8_t* lb = (const uint8_t*)p.kv_nope + ((int64_t)pg * p.kv_sp + tok * kv_st);
        const uint16_t* rb = p.kv_rope + ((int64_t)pg * p.kr_sp + tok * kr_st);
        const float* scb = p.kv_scale + ((int64_t)pg * p.ks_sp + tok);
        const int left = L - st * kStageTok;
        issue_stage8<NL>(ring + (k % NSTAGE) * kSB, lb, rb, scb, kv_st, kr_st, p.ks_sb,
                         (left < kStageTok ? left : kStageTok) - 1, NL == 1 ? 0 : wave, lane);
        return;
      }
      const uint16_t* nb;
      const uint16_t* rb;
      if (paged) {
        const int pidx = st >> 1;
        if (pidx - pbase >= 64) load_page_ids(pidx);  // uniform
        const int pg = __builtin_amdgcn_readlane(bt_lane, pidx - pbase);
        const int tok = (st & 1) * kStageTok;
        nb = p.kv_nope + ((int64_t)pg * p.kv_sp + tok * kv_st);
        rb = p.kv_rope + ((int64_t)pg * p.kr_sp + tok * kr_st);
      } else {
        nb = p.kv_nope + ((int64_t)b * p.kv_sb + (int64_t)st * kStageTok * kv_st);
        rb = p.kv_rope + ((int64_t)b * p.kr_sb + (int64_t)st * kStageTok * kr_st);
      }
      const int left = L - st * kStageTok;
      issue_stage<NL>(ring + (k % NSTAGE) * kSB, nb, rb, kv_st, kr_st,
                      (left < kStageTok ? left : kStageTok) - 1, NL == 1 ? 0 : wave, lane);
    };

    // kProg: the loads of issue_stage<1> for stage k, in parts: prog_prepare forms the bases
    // and per-lane offsets once, prog_rope issues the four rope blocks, prog_seg(s) the four
    // blocks of latent segment s (block q*9 + s: rows 8q .. 8q+7, chunks 8s .. 8s+7)
    // fp8 cache (KV8, paged only): the loads of issue_stage8<1>, the latent in four 128-dim
    // blocks (prog_seg(s): block s of the four row groups and the stage's 32 scales of block s)
    // sparse (bf16/fp16): each of the lane's four token rows has its own address (sn, sr)
    const auto uni64 = [](const char* q) __attribute__((always_inline)) {
      const uint64_t v = (uint64_t)(uintptr_t)q;
      return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32)) << 32) |
             (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    };
    const auto ring_base = [&]() __attribute__((always_inline)) {
      return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)ring);
    };
    struct ProgLoads {
      const char* nb;
      const uint16_t* rb;
      const float* scb;
      uint32_t on[4], orp[4];
      const char* sn[SPARSE ? 4 : 1];
      const char* sr[SPARSE ? 4 : 1];
    };
    auto prog_prepare = [&](int k) __attribute__((always_inline)) {
      ProgLoads r;
      r.scb = nullptr;
      const int st = st_begin + k;
      if constexpr (SPARSE) {  // as issue_stage_sparse<1>
        const int valid_rows = (L - st * kStageTok) < kStageTok ? L - st * kStageTok : kStageTok;
        const int32_t LDS_AS* idx_stage = (const int32_t LDS_AS*)idx_sh + k * kStageTok;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int rr = 8 * q + (lane >> 3);
          const int t = rr < valid_rows ? rr : valid_rows - 1;
          int64_t idx = idx_stage[t];
          if (idx < 0 || idx >= p.pool_tokens) idx = 0;
          const int64_t pg = idx >> 6, rw = idx & 63;
          const uint32_t cl = (uint32_t)(((lane & 7) ^ stage_swz(((q & 1) << 3) | (lane >> 3))) << 4);
          r.sn[q] = (const char*)(p.kv_nope + pg * p.kv_sp + rw * p.kv_st) + cl;
          r.sr[q] = (const char*)(p.kv_rope + pg * p.kr_sp + rw * p.kr_st) + cl;
        }
        return r;
      }
      if (paged) {
        const int pidx = st >> 1;
        if (pidx - pbase >= 64) load_page_ids(pidx);  // uniform
        const int pg = __builtin_amdgcn_readlane(bt_lane, pidx - pbase);
        const int tok = (st & 1) * kStageTok;
        if constexpr (KV8) {
          r.nb = (const char*)p.kv_nope + ((int64_t)pg * p.kv_sp + tok * kv_st);
          r.scb = p.kv_scale + ((int64_t)pg * p.ks_sp + tok);
        } else {
          r.nb = (const char*)(p.kv_nope + ((int64_t)pg * p.kv_sp + tok * kv_st));
        }
        r.rb = p.kv_rope + ((int64_t)pg * p.kr_sp + tok * kr_st);
      } else {
        r.nb = (const char*)(p.kv_nope + ((int64_t)b * p.kv_sb + (int64_t)st * kStageTok * kv_st));
        r.rb = p.kv_rope + ((int64_t)b * p.kr_sb + (int64_t)st * kStageTok * kr_st);
      }
      const int left = L - st * kStageTok;
      const int last_row = (left < kStageTok ? left : kStageTok) - 1;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int rr = 8 * q + (lane >> 3);  // LDS row
        const int row = rr < last_row ? rr : last_row;  // rows past the sequence end re-read its last row
        if constexpr (KV8) {
          r.on[q] = (uint32_t)(row * kv_st) + (uint32_t)(((lane & 7) ^ swz8(rr)) << 4);
          r.orp[q] = (uint32_t)(row * kr_st) * 2 + (uint32_t)(((lane & 7) ^ swzr(rr)) << 4);
        } else {
          const uint32_t cl = (uint32_t)(((lane & 7) ^ stage_swz(((q & 1) << 3) | (lane >> 3))) << 4);
          r.on[q] = (uint32_t)(row * kv_st) * 2 + cl;
          r.orp[q] = (uint32_t)(row * kr_st) * 2 + cl;
        }
      }
      return r;
    };
    auto prog_rope = [&](const ProgLoads& r) __attribute__((always_inline)) {
      if constexpr (SPARSE) {
#pragma unroll
        for (int q = 0; q < 4; ++q) dma16_lane(r.sr[q], (uint32_t)(uintptr_t)(ring + (q * 9 + 8) * 1024));
        return;
      }
      if constexpr (!KV8) {  // block q*9 + 8: one scalar instruction per load
        const uint64_t rb = uni64((const char*)r.rb);
        const uint32_t rs = ring_base();
        dma16_m0<8 * 1024, 0, true>(rb, r.orp[0], rs);
        dma16_m0<17 * 1024, 0, true>(rb, r.orp[1], rs);
        dma16_m0<26 * 1024, 0, true>(rb, r.orp[2], rs);
        dma16_m0<35 * 1024, 0, true>(rb, r.orp[3], rs);
        return;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        dma16(r.rb, r.orp[q], (uint32_t)(uintptr_t)(ring + (KV8 ? kRopeOff8 + q * 1024 : (q * 9 + 8) * 1024)));
    };
    auto prog_seg = [&](const ProgLoads& r, int sgm) __attribute__((always_inline)) {
      if constexpr (SPARSE) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          dma16_lane(r.sn[q] + 128 * sgm, (uint32_t)(uintptr_t)(ring + (q * 9 + sgm) * 1024));
      } else if constexpr (KV8) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          dma16(r.nb + 128 * sgm, r.on[q], (uint32_t)(uintptr_t)(ring + (q * 4 + sgm) * 1024));
        dma16(r.scb + sgm * p.ks_sb, (uint32_t)((lane & 7) << 4), (uint32_t)(uintptr_t)(ring + kScaleOff8 + sgm * 1024));
      } else {  // block q*9 + sgm, the global address stepped by the instruction offset
        const uint64_t nb = uni64(r.nb);
        const uint32_t rs = ring_base();
        switch (sgm) {  // a constant once the loops around the call are unrolled
#define MLA_SEG(S)                                                     \
  case S:                                                              \
    dma16_m0<(S) * 1024, 128 * (S), true>(nb, r.on[0], rs);           \
    dma16_m0<(9 + (S)) * 1024, 128 * (S), true>(nb, r.on[1], rs);     \
    dma16_m0<(18 + (S)) * 1024, 128 * (S), true>(nb, r.on[2], rs);    \
    dma16_m0<(27 + (S)) * 1024, 128 * (S), true>(nb, r.on[3], rs);    \
    break;
          MLA_SEG(0) MLA_SEG(1) MLA_SEG(2) MLA_SEG(3) MLA_SEG(4) MLA_SEG(5) MLA_SEG(6) default: MLA_SEG(7)
#undef MLA_SEG
        }
      }
    };

    // One pass over the segment's stages.  Returns true (uniformly across the workgroup)
    // when a first-stage-reference pass saw a score above its reference by more than tau.
    auto run_pass = [&](auto mode_tag) __attribute__((always_inline)) -> bool {
      constexpr int MODE = decltype(mode_tag)::value;
      if constexpr (MODE != kPassRowMax) {
#pragma unroll
        for (int dt = 0; dt < kDimTiles; ++dt)
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) o[dt][ht] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) l_part[ht] = l_exact[ht] = 0.f;
      }
      if constexpr (MODE != kPassFixedRef) {
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) m_ref[ht] = -INFINITY;
      }
      if constexpr (MODE == kPassFirstStageRef && !WS) {
        if (wave == 0) over_sh[lane & 3] = 0;  // uniform branch; ordered by the first barriers
        wait_lgkm0();
      }
      // the first pass uses the page ids loaded in the prologue; a pass after an abort reloads
      // the window the segment starts in.  The compiler's wait for the ids (and the stage
      // waits, for the query fragments) count only the loads issued after them.
      if (pbase != page) load_page_ids(page);  // uniform

      if constexpr (NSTAGE == 1) {
        if (k0 < nst) issue(k0);
      } else {
#pragma unroll
        for (int k = 0; k < LEAD; ++k)
          if (k < nst) issue(k);
      }
      // One LDS buffer (NSTAGE == 1): the next stage is loaded into it once every wave
      // sharing it has consumed the current one; latency is hidden by the other waves of the
      // CU instead.
      auto refill_single = [&](int k) __attribute__((always_inline)) {
        if constexpr (NSTAGE == 1 && !(kProg && MODE != kPassRowMax)) {
          if constexpr (NW > 1 && !WS) lds_barrier();
          if (k + kStep < nst) issue(k + kStep);
        }
      };

      // ---- O^T += V^T P^T over the 32 tokens of stage kp; DV fragments in flight
      auto v_base = [&](int kp) __attribute__((always_inline)) {
        const uint8_t LDS_AS* vb = (kDeq ? deq : ring + (kp % NSTAGE) * kSB) + v_lane;
        asm volatile("" : "+v"(vb));
        return vb;
      };
      // Tiles go in d4-major order, t = 8*d4 + s for dim tile dt = 4s + d4, so the XOR of the
      // lane address changes once per eight tiles.
      auto v_frag = [&](const uint8_t LDS_AS* vb, int t) __attribute__((always_inline)) {
        const uint8_t LDS_AS* xb =
            (t >> 3) ? (const uint8_t LDS_AS*)(uintptr_t)((uint32_t)(uintptr_t)vb ^ (uint32_t)(32 * (t >> 3))) : vb;
        return lds_tr_pair(xb + (t & 7) * 1024);
      };
      // the first DV V^T fragments of stage kp (issued ahead of the softmax to hide latency)
      // kProg: tiles in segment-major order (dt = t), so segment s is read by tiles 4s .. 4s+3
      // and refilled (`seg`) once the last of them has issued: every read of it has landed,
      // since each fragment is awaited before the MFMA that takes it
      auto v_frag_s = [&](const uint8_t LDS_AS* vb, int t) __attribute__((always_inline)) {
        const uint8_t LDS_AS* xb =
            (t & 3) ? (const uint8_t LDS_AS*)(uintptr_t)((uint32_t)(uintptr_t)vb ^ (uint32_t)(32 * (t & 3))) : vb;
        return lds_tr_pair(xb + (t >> 2) * 1024);
      };
      auto v_prefetch = [&](int kp, i32x4 (&vf)[DV]) __attribute__((always_inline)) {
        const uint8_t LDS_AS* vb = v_base(kp);
#pragma unroll
        for (int n = 0; n < DV; ++n) vf[n] = kProg ? v_frag_s(vb, n) : v_frag(vb, n);
      };
      auto pv_stage = [&](int kp, i32x4 (&pb)[HT], i32x4 (&vf)[DV], auto prog_tag, const auto& seg)
                          __attribute__((always_inline)) {
        constexpr bool kP = decltype(prog_tag)::value;
        const uint8_t LDS_AS* vb = v_base(kp);
#pragma unroll
        for (int t = 0; t < kDimTiles; ++t) {
          const int dt = kP ? t : 4 * (t & 7) + (t >> 3);
          const i32x4 a = vf[t % DV];
          if (t + DV < kDimTiles) vf[t % DV] = kP ? v_frag_s(vb, t + DV) : v_frag(vb, t + DV);
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) o[dt][ht] = mfma32<DT>(a, pb[ht], o[dt][ht]);
          if constexpr (kP) {
            if ((t & 3) == 3) seg(t >> 2);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        // The last MFMAs are still reading their A/B operands (P^T and the last V^T fragment)
        // over several passes after they issue.  The compiler's hazard model lets a VALU write
        // reuse those registers a few cycles later (seen corrupting the last dim tile of the
        // second row tile), so hold them for 32 wait states: the asm ties the operands, so no
        // write to their registers can be placed before it.
        operand_guard<HT>(pb, vf[(kDimTiles - 1) % DV]);
      };
      // fp8 cache: V^T fragment t (natural dim-tile order) as raw codes, converted at use
      auto v8_base = [&](int kp) __attribute__((always_inline)) {
        const uint8_t LDS_AS* vb = ring + (kp % NSTAGE) * kSB + v8_lane;
        asm volatile("" : "+v"(vb));
        return vb;
      };
      auto v8_raw = [&](const uint8_t LDS_AS* vb, int t) __attribute__((always_inline)) {
        const uint8_t LDS_AS* xb =
            (t & 7) ? (const uint8_t LDS_AS*)(uintptr_t)((uint32_t)(uintptr_t)vb ^ (uint32_t)(16 * (t & 7))) : vb;
        return __builtin_amdgcn_ds_read_tr8_b64_v2i32((i32x2 LDS_AS*)(xb + 1024 * (t >> 3)));
      };
      auto v8_prefetch = [&](int kp, i32x2 (&vr)[DV]) __attribute__((always_inline)) {
        const uint8_t LDS_AS* vb = v8_base(kp);
#pragma unroll
        for (int n = 0; n < DV; ++n) vr[n] = v8_raw(vb, n);
      };
      // O^T += V^T (P^T * s): the scales of V (per token and 128-dim block) multiply P^T, once
      // per block of eight dim tiles.  On the sequence's last stage the scales of rows past its
      // end are not data (their P is 0): they are replaced by 0 so that 0 * s stays 0.
      // kProg: `seg(b)` after the last MFMA of 128-dim block b (its V^T codes and scales have
      // all been read by then: each tile's codes are converted, and each block's scales taken,
      // before the MFMAs that use them)
      auto pv_stage8 = [&](int kp, const float (&pvf)[HT][8], i32x2 (&vr)[DV], const auto& seg)
                           __attribute__((always_inline)) {
        const uint8_t LDS_AS* vb = v8_base(kp);
        const uint8_t LDS_AS* scb = ring + (kp % NSTAGE) * kSB + kScaleOff8 + 16 * g;
        const int left = L - (st_begin + kp) * kStageTok;
        // P^T * s for 128-dim block bk
        auto make_pb = [&](int bk, i32x4 (&pbo)[HT]) __attribute__((always_inline)) {
          f32x4 s0 = *(const f32x4 LDS_AS*)(scb + bk * 1024);       // tokens 4g .. 4g+3
          f32x4 s1 = *(const f32x4 LDS_AS*)(scb + bk * 1024 + 64);  // tokens 16+4g ..
          if (left < kStageTok) {  // uniform
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              s0[i] = 4 * g + i < left ? s0[i] : 0.f;
              s1[i] = 16 + 4 * g + i < left ? s1[i] : 0.f;
            }
          }
#pragma unroll
          for (int ht = 0; ht < HT; ++ht)
            pbo[ht] = i32x4{(int)pack2<DT>(pvf[ht][0] * s0[0], pvf[ht][1] * s0[1]),
                            (int)pack2<DT>(pvf[ht][2] * s0[2], pvf[ht][3] * s0[3]),
                            (int)pack2<DT>(pvf[ht][4] * s1[0], pvf[ht][5] * s1[1]),
                            (int)pack2<DT>(pvf[ht][6] * s1[2], pvf[ht][7] * s1[3])};
        };
        // As in the QK loop: the operands of tile t+1 (V^T conversion, and P^T * s at a block
        // start) are produced before MFMA t issues, and the operands of tile t-1 stay live until
        // MFMA t has issued.
        i32x4 pbb[HT], pbb_old[HT];
        make_pb(0, pbb);
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) pbb_old[ht] = pbb[ht];
        i32x4 a_cur = cvt_fp8x8(vr[0], 1.0f);
        vr[0] = v8_raw(vb, DV);
        i32x4 a_prev = a_cur;
#pragma unroll
        for (int t = 0; t < kDimTiles; ++t) {
          i32x4 a_next = a_cur;
          i32x4 pbb_next[HT];
          const bool new_block = t + 1 < kDimTiles && ((t + 1) & 7) == 0;
          if (t + 1 < kDimTiles) {
            a_next = cvt_fp8x8(vr[(t + 1) % DV], 1.0f);
            if (t + 1 + DV < kDimTiles) vr[(t + 1) % DV] = v8_raw(vb, t + 1 + DV);
          }
          if (new_block) make_pb((t + 1) >> 3, pbb_next);
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) o[t][ht] = mfma32<DT>(a_cur, pbb[ht], o[t][ht]);
          if constexpr (kProg) {
            if ((t & 7) == 7) seg(t >> 3);
          }
          asm volatile("" ::"v"(a_prev));
          if ((t & 7) == 0 && t > 0) {
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) asm volatile("" ::"v"(pbb_old[ht]));
          }
          __builtin_amdgcn_sched_barrier(0);
          a_prev = a_cur;
          a_cur = a_next;
          if (new_block) {
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) {
              pbb_old[ht] = pbb[ht];
              pbb[ht] = pbb_next[ht];
            }
          }
        }
        operand_guard<HT>(pbb, a_prev);
      };

      bool abort = false;
      // wave-split: this wave's own "score above reference" flag of its previous stage
      bool over_prev = false;
#pragma unroll 1
      for (int j = 0, k = k0; k < nst; ++j, k += kStep) {  // j: the wave's own stage count
        const int remaining_after = nst - 1 - k;
        // kProg after the first own stage: the stage came in the order rope, segment 0, ..,
        // segment 7 (four loads each), so QK starts once the rope and segment 0 have landed
        // and waits for segment s only before its first fragment read (prog_wait)
        constexpr bool kProgWait = kProg && !KV8 && MODE != kPassRowMax;
        const bool prog_wait = kProgWait && j > 0;  // uniform
        if (prog_wait) {
          wait_vmcnt<28>();
        } else {
          wait_stage<kLPS / NL, NSTAGE>(remaining_after < LEAD - 1 ? remaining_after : LEAD - 1);
        }
        if constexpr (!WS) lds_barrier();
        // the previous stage's flags, read now and tested after this stage's QK product
        int prev_over = 0;
        if constexpr (MODE == kPassFirstStageRef) {
          if constexpr (WS) {
            prev_over = over_prev;
          } else {
            if (k > 0) prev_over = over_sh[(k - 1) & 3];
            if (k > 1 && wave == 0) over_sh[(k - 2) & 3] = 0;  // uniform branch
          }
        }
        if constexpr (NSTAGE > 1) {
          if (k + LEAD < nst) issue(k + LEAD);
        }

        if constexpr (kDeq) {
          // dequantise this wave's row group of stage k into the bf16 stage (its layout: row r,
          // 16-byte chunk c of 64-dim segment s in block (r/8)*9 + s, slot 8(r%8) + (c ^ swz));
          // rows past the sequence end take the last row's scales (their codes are its copies)
          const uint8_t LDS_AS* f8 = ring + (k % NSTAGE) * kSB;
          const int r = 8 * wave + (lane >> 3);
          const int left = L - (st_begin + k) * kStageTok;
          const int rs = r < left ? r : left - 1;
          const int c = (lane & 7) ^ stage_swz(r & 15);
          float sc[4];
#pragma unroll
          for (int b4 = 0; b4 < 4; ++b4) sc[b4] = *(const float LDS_AS*)(f8 + kScaleOff8 + b4 * 1024 + 4 * rs);
#pragma unroll
          for (int sg = 0; sg < 8; ++sg) {
            const int c16 = 4 * (sg & 1) + (c >> 1);
            const i32x2 raw = *(const i32x2 LDS_AS*)(f8 + (4 * wave + (sg >> 1)) * 1024 +
                                                     16 * (8 * (r & 7) + (c16 ^ swz8(r))) + 8 * (c & 1));
            *(i32x4 LDS_AS*)(deq + (9 * wave + sg) * 1024 + 16 * lane) = cvt_fp8x8(raw, sc[sg >> 1]);
          }
          *(i32x4 LDS_AS*)(deq + (9 * wave + 8) * 1024 + 16 * lane) =
              *(const i32x4 LDS_AS*)(f8 + kRopeOff8 + wave * 1024 + 16 * (8 * (r & 7) + (c ^ swzr(r))));
          wait_lgkm0();
          lds_barrier();
        }
        const uint8_t LDS_AS* sb = kDeq ? (const uint8_t LDS_AS*)deq : ring + (k % NSTAGE) * kSB;
        const int st = st_begin + k;

        // ---- S^T = K Q^T over 576 dims: two 16-token tiles x HT 16-row tiles.
        // Fragment n = 2*kk + tt; DK fragments in flight ahead of the MFMAs.
        f32x4 acc[HT][2];
        i32x4 kf[DK];
        // per-stage lane bases; the empty asm stops the compiler from precomputing one
        // address register per fragment (the fragment offsets below fit the DS immediate)
        const uint8_t LDS_AS* kb0 = sb + k_lane0;
        const uint8_t LDS_AS* kb1 = sb + k_lane1;
        asm volatile("" : "+v"(kb0));
        asm volatile("" : "+v"(kb1));
#define MLA_KFRAG(N) \
  (*(const i32x4 LDS_AS*)((((N) >> 1) & 1 ? kb1 : kb0) + ((N) & 1) * kPanelBytes + ((N) >> 2) * 1024))
        // fp8: the K scales of rows li and 16 + li, per 128-dim block
        float sk[2][4];
        const uint8_t LDS_AS* kbl = sb + kb8;
        const uint8_t LDS_AS* kbr = sb + kr8;
        if constexpr (kInl8) {
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int bk = 0; bk < 4; ++bk)
              sk[tt][bk] = *(const float LDS_AS*)(sb + kScaleOff8 + bk * 1024 + 4 * (16 * tt + li));
          asm volatile("" : "+v"(kbl));
          asm volatile("" : "+v"(kbr));
        }
        // fp8 fragment n = 2*kk + tt as raw data: 8 codes (latent) or 8 bf16 values (rope)
        auto k8_raw = [&](int n) __attribute__((always_inline)) -> i32x4 {
          const int kk = n >> 1, tt = n & 1;
          if (kk < 16) {
            const uint32_t x = (uint32_t)((32 * (kk & 3)) ^ (64 * tt));  // bits 5-6 only
            const uint8_t LDS_AS* a = x ? (const uint8_t LDS_AS*)(uintptr_t)((uint32_t)(uintptr_t)kbl ^ x) : kbl;
            const i32x2 r = *(const i32x2 LDS_AS*)(a + 8192 * tt + 1024 * (kk >> 2));
            const int r0 = r.x, r1 = r.y;
            return i32x4{r0, r1, 0, 0};
          }
          const uint8_t LDS_AS* a =
              kk == 16 ? kbr : (const uint8_t LDS_AS*)(uintptr_t)((uint32_t)(uintptr_t)kbr ^ 64u);
          return *(const i32x4 LDS_AS*)(a + 2048 * tt);
        };
        if constexpr (kInl8) {
          // The converted fragments are VALU results read by the (inline-asm) MFMAs, whose
          // hazards the compiler does not see.  Fragment n+1 is converted before MFMA n issues
          // (so an MFMA separates every conversion from its reader), and fragment n-1 is held
          // live until MFMA n has issued (so no conversion overwrites the operands of the MFMA
          // just issued).
          auto k8_conv = [&](int n, const i32x4& raw) __attribute__((always_inline)) -> i32x4 {
            if ((n >> 1) < 16) {
              const int r0 = raw.x, r1 = raw.y;
              return cvt_fp8x8(i32x2{r0, r1}, sk[n & 1][n >> 3]);
            }
            return raw;
          };
#pragma unroll
          for (int n = 0; n < DK; ++n) kf[n] = k8_raw(n);
          i32x4 c_cur = k8_conv(0, kf[0]);
          kf[0] = k8_raw(DK);
          i32x4 c_prev = c_cur;
#pragma unroll
          for (int n = 0; n < 2 * kKSteps; ++n) {
            i32x4 c_next = c_cur;
            if (n + 1 < 2 * kKSteps) {
              c_next = k8_conv(n + 1, kf[(n + 1) % DK]);
              if (n + 1 + DK < 2 * kKSteps) kf[(n + 1) % DK] = k8_raw(n + 1 + DK);
            }
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) {
              if (n < 2)
                mfma_qk_first<DT>(acc[ht][n & 1], c_cur, qf[ht][n >> 1]);
              else
                mfma_qk<DT>(acc[ht][n & 1], c_cur, qf[ht][n >> 1]);
            }
            asm volatile("" ::"v"(c_prev));
            __builtin_amdgcn_sched_barrier(0);
            c_prev = c_cur;
            c_cur = c_next;
          }
        } else {
          // fragment m reads latent segment m / 4 (the rope for m >= 32); the loads of segment
          // s are awaited before fragment 4s is read (outstanding: the four loads of each later
          // segment).  In a wave's first own stage nothing is in flight during QK (the stage was
          // awaited whole and the next one is issued after QK), so the waits cost nothing there.
          auto seg_wait = [&](int m) __attribute__((always_inline)) {
            if constexpr (kProgWait) {
              if ((m & 3) == 0 && m >= 4 && m < 32) {
                switch (m >> 2) {
                  case 1: wait_vmcnt<24>(); break;
                  case 2: wait_vmcnt<20>(); break;
                  case 3: wait_vmcnt<16>(); break;
                  case 4: wait_vmcnt<12>(); break;
                  case 5: wait_vmcnt<8>(); break;
                  case 6: wait_vmcnt<4>(); break;
                  default: wait_vmcnt<0>(); break;
                }
              }
            }
          };
#pragma unroll
          for (int n = 0; n < DK; ++n) {
            seg_wait(n);
            kf[n] = MLA_KFRAG(n);
          }
#pragma unroll
          for (int n = 0; n < 2 * kKSteps; ++n) {
            const i32x4 a = kf[n % DK];
            if (n + DK < 2 * kKSteps) {
              seg_wait(n + DK);
              kf[n % DK] = MLA_KFRAG(n + DK);
            }
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) {
              if (n < 2)
                mfma_qk_first<DT>(acc[ht][n & 1], a, qf[ht][n >> 1]);
              else
                mfma_qk<DT>(acc[ht][n & 1], a, qf[ht][n >> 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
#undef MLA_KFRAG
        qk_settle(acc[0][0]);
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
          if (ht > 0) qk_touch(acc[ht][0]);
          qk_touch(acc[ht][1]);
        }
        if constexpr (MODE == kPassFirstStageRef) {
          if (prev_over) {  // uniform: every wave read the same flags after the same barrier
            abort = true;
            break;
          }
        }
        i32x4 vf[DV];
        i32x2 vr[DV];
        if constexpr (MODE != kPassRowMax) {
          if constexpr (kInl8) v8_prefetch(k, vr);
          else v_prefetch(k, vf);
        }
        // kProg: the next own stage's loads, rope now (QK has read it), latent during PV
        const bool prog_next = kProg && MODE != kPassRowMax && k + kStep < nst;  // uniform
        ProgLoads prog{};
        if constexpr (kProg && MODE != kPassRowMax) {
          if (prog_next) {
            prog = prog_prepare(k + kStep);
            prog_rope(prog);
          }
        }

        // ---- sparse: mask the stage's tokens whose index is past the list or outside the pool
        if constexpr (SPARSE) {
          const int left = L - st * kStageTok;
          bool valid = false;
          if (lane < kStageTok && lane < left) {
            const int v = ((const int32_t LDS_AS*)idx_sh)[k * kStageTok + lane];
            valid = v >= 0 && (int64_t)v < p.pool_tokens;
          }
          const uint32_t vmask = (uint32_t)__builtin_amdgcn_ballot_w64(valid);
#pragma unroll
          for (int ht = 0; ht < HT; ++ht)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (!((vmask >> (16 * tt + 4 * g + r)) & 1u)) acc[ht][tt][r] = -INFINITY;
        }
        // ---- mask tokens past each row's limit (sequence tail / causal)
        if (!SPARSE && st * kStageTok + kStageTok > lmin) {
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) {
            // token 16*tt + 4*g + r of the stage is visible iff 16*tt + r < rel; the empty
            // asm keeps the compiler from hoisting one precomputed limit per (tt, r) out of
            // the loop (that costs a register each)
            int rel = lim[ht] - st * kStageTok - 4 * g;
            asm volatile("" : "+v"(rel));
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (16 * tt + r >= rel) acc[ht][tt][r] = -INFINITY;
          }
        }

        // ---- this lane's largest scaled score per row tile
        float lmx[HT];
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
          const float v = max3f(max3f(acc[ht][0][0], acc[ht][0][1], acc[ht][0][2]),
                                max3f(acc[ht][0][3], acc[ht][1][0], acc[ht][1][1]),
                                max3f(acc[ht][1][2], acc[ht][1][3], -INFINITY));
          lmx[ht] = v * p.scale_log2;
        }
        if constexpr (MODE == kPassRowMax) {
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) m_ref[ht] = fmaxf(m_ref[ht], lmx[ht]);
          refill_single(k);
          continue;
        }
        if constexpr (MODE == kPassFirstStageRef) {
          if (WS ? j == 0 : k == 0) {
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) m_ref[ht] = wave_max_g(lmx[ht]);
          } else {
            bool over = false;
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) over |= lmx[ht] > m_ref[ht] + kTau;
            if constexpr (WS) {
              over_prev = __builtin_amdgcn_ballot_w64(over) != 0;
            } else {
              if (__builtin_amdgcn_ballot_w64(over) != 0) over_sh[k & 3] = 1;  // uniform branch
            }
          }
        }

        // ---- P^T = 2^(S^T * sm_scale * log2(e) - m), packed to the B operand of PV
        i32x4 pb[HT];
        float pvf[HT][8];  // fp8: P kept in fp32 until the per-block scales are applied
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
          const float mu = m_ref[ht] == -INFINITY ? 0.f : m_ref[ht];
          float pv[2][4];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) pv[tt][r] = fast_exp2(acc[ht][tt][r] * p.scale_log2 - mu);
          // P rounded to the 16-bit type as the PV product takes it; the row sum counts those
          // rounded values (a sum of the unrounded ones would leave the weights on V summing
          // to 1 + O(2^-9): with V far from zero on average that bias does not cancel)
          const i32x4 pr = i32x4{(int)pack2<DT>(pv[0][0], pv[0][1]), (int)pack2<DT>(pv[0][2], pv[0][3]),
                                 (int)pack2<DT>(pv[1][0], pv[1][1]), (int)pack2<DT>(pv[1][2], pv[1][3])};
          l_part[ht] = packed_sum<DT>(pr, l_part[ht]);
          l_exact[ht] += ((pv[0][0] + pv[0][1]) + (pv[0][2] + pv[0][3])) +
                         ((pv[1][0] + pv[1][1]) + (pv[1][2] + pv[1][3]));
          if constexpr (kInl8) {
            // the V scales are powers of two: P * scale rounds to exactly this P times the scale
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t x = (uint32_t)pr[j];
              pvf[ht][2 * j] = __uint_as_float(x << 16);
              pvf[ht][2 * j + 1] = __uint_as_float(x & 0xffff0000u);
            }
          } else {
            pb[ht] = pr;
          }
        }

        if constexpr (kInl8) {
          pv_stage8(k, pvf, vr, [&](int blk) __attribute__((always_inline)) {
            if (prog_next) prog_seg(prog, blk);
          });
        } else if constexpr (kProg) {
          pv_stage(k, pb, vf, std::true_type{}, [&](int sgm) __attribute__((always_inline)) {
            if (prog_next) prog_seg(prog, sgm);
          });
        } else {
          pv_stage(k, pb, vf, std::false_type{}, [](int) {});
        }
        refill_single(k);
        if constexpr (MODE == kPassFirstStageRef && !WS) wait_lgkm0();  // flag store lands before the barrier
      }
      if constexpr (MODE == kPassFirstStageRef) {
        if constexpr (WS) {
          if (!abort) abort = over_prev;  // the wave's last stage's flag
        } else {
          if (!abort && nst > 1) {  // the last stage's flags
            lds_barrier();
            abort = over_sh[(nst - 1) & 3] != 0;
          }
        }
      }
      wait_vmcnt<0>();  // an abandoned pass may leave stage loads in flight
      // every wave is done with the LDS ring before it is refilled (a wave-split slot has one
      // user)
      if constexpr (!WS) lds_barrier();
      return abort;
    };

    if (run_pass(std::integral_constant<int, kPassFirstStageRef>{})) {
      run_pass(std::integral_constant<int, kPassRowMax>{});
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) m_ref[ht] = wave_max_g(m_ref[ht]);
      run_pass(std::integral_constant<int, kPassFixedRef>{});
    }

    // ---- epilogue: finish the row sums, normalise, write final or partial output.
    // Branch-free on purpose (only uniform branches): at a divergent join the register
    // allocator has placed the AGPR -> VGPR reload of an output tile in a block still running
    // with a narrowed exec mask, so lanes outside it lost that tile.  Instead, lanes of
    // padding rows (past the last row) store to the last row: their query was clamped to that
    // row, so they computed bitwise the same values; and all four lane groups of a row store
    // its lse (the same value).
    const int slot0 = __builtin_amdgcn_readfirstlane(slot_lo_v);
    const bool single = (__builtin_amdgcn_readfirstlane(slot_hi_v) - slot0) == 1;
    if constexpr (WS) {
      // ---- wave-split merge.  Wave w holds (m_w, l_w, O_w) over its stages (m_w = -inf and
      // l_w = 0 for a wave that had none); the segment's result is
      //   O = sum_w 2^(m_w - m) O_w / lsum,  lsum = sum_w 2^(m_w - m) l_w,  m = max_w m_w,
      // and lse = m + log2(xsum) with xsum the same sum over the waves' fp32 row sums (log2
      // units, as every split's lse).  Each wave scales its O_w
      // into LDS (fp32 rows of 512 with a 16-byte pad: conflict-free 16-byte stores), then
      // wave w sums and stores dims 128w .. 128w + 127 of all 16 rows.  The slots are free:
      // every wave waited for its own stage loads before the first barrier.
      static_assert(kMergeBytes <= kSmem, "merge staging exceeds the shared memory");
      const int64_t slot = slot0 + split;
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) {
        const float l_w = wave_sum_g(l_part[ht]);
        const float x_w = wave_sum_g(l_exact[ht]);
        if (g == 0) {
          merge_sh[wave][0][li] = m_ref[ht];
          merge_sh[wave][1][li] = l_w;
          merge_sh[wave][2][li] = x_w;
        }
        wait_lgkm0();
        lds_barrier();
        float m = -INFINITY;
#pragma unroll
        for (int v = 0; v < NW; ++v) m = fmaxf(m, merge_sh[v][0][li]);
        float lsum = 0.f, xsum = 0.f, c = 0.f;
#pragma unroll
        for (int v = 0; v < NW; ++v) {
          const float mv = merge_sh[v][0][li];
          const float sv = mv == -INFINITY ? 0.f : fast_exp2(mv - m);
          lsum += sv * merge_sh[v][1][li];
          xsum += sv * merge_sh[v][2][li];
          if (v == wave) c = sv;  // uniform
        }
        c *= lsum > 0.f ? 1.f / lsum : 0.f;
        uint8_t LDS_AS* mine = smem + (wave * 16 + li) * kMergePitch + 16 * g;
#pragma unroll
        for (int dt = 0; dt < kDimTiles; ++dt) {  // O_w^T tile dt: row li, dims 16dt + 4g ..
          *(f32x4 LDS_AS*)(mine + 64 * dt) = o[dt][ht] * c;
          __builtin_amdgcn_sched_barrier(0);
        }
        wait_lgkm0();
        lds_barrier();
        // lane (q, cc) = (lane / 16, lane % 16): rows q, q + 4, q + 8, q + 12, dims
        // 128w + 4cc .. + 3 and 128w + 64 + 4cc .. + 3 (16 lanes read 256 contiguous bytes:
        // conflict-free).  Padding rows store the last row's (identical) values.
        const int cc = lane & 15, q = lane >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = q + 4 * i;
          f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll
          for (int v = 0; v < NW; ++v) {
            const uint8_t LDS_AS* src = smem + (v * 16 + r) * kMergePitch + (128 * wave + 4 * cc) * 4;
            a0 += *(const f32x4 LDS_AS*)src;
            a1 += *(const f32x4 LDS_AS*)(src + 256);
          }
          int row = row0 + 16 * ht + r;
          row = row < p.rows ? row : p.rows - 1;
          if (single) {  // uniform: the final output, rounded once to the input dtype
            const int s = row / p.heads;
            const int h = row - s * p.heads;
            uint16_t* d = p.out + (b * p.o_sb + s * p.o_ss + h * p.o_sh) + 128 * wave + 4 * cc;
            *(i32x2*)d = i32x2{(int)pack2<DT>(a0[0], a0[1]), (int)pack2<DT>(a0[2], a0[3])};
            *(i32x2*)(d + 64) = i32x2{(int)pack2<DT>(a1[0], a1[1]), (int)pack2<DT>(a1[2], a1[3])};
          } else if (p.part16) {  // uniform: 16-bit partials (the reference's own format)
            uint16_t* d = p.ws_o + (slot * p.rows + row) * kDV + 128 * wave + 4 * cc;
            *(i32x2*)d = i32x2{(int)pack2<DT>(a0[0], a0[1]), (int)pack2<DT>(a0[2], a0[3])};
            *(i32x2*)(d + 64) = i32x2{(int)pack2<DT>(a1[0], a1[1]), (int)pack2<DT>(a1[2], a1[3])};
          } else {  // the split's scaled fp16 partial: chunk `wave` of row r spans lanes cc
            float am = fmaxf(amax4(a0), amax4(a1));
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) am = fmaxf(am, __shfl_xor(am, off));
            const int e = part_exp(am);
            const f32x4 b0 = a0 * exp2i(e), b1 = a1 * exp2i(e);
            uint16_t* d = p.ws_o + (slot * p.rows + row) * kDV + 128 * wave + 4 * cc;
            *(i32x2*)d = i32x2{(int)pack2<MLA_DTYPE_F16>(b0[0], b0[1]), (int)pack2<MLA_DTYPE_F16>(b0[2], b0[3])};
            *(i32x2*)(d + 64) = i32x2{(int)pack2<MLA_DTYPE_F16>(b1[0], b1[1]), (int)pack2<MLA_DTYPE_F16>(b1[2], b1[3])};
            p.ws_scale[(slot * p.rows + row) * 4 + wave] = exp2i(-e);  // 16 lanes, one value
          }
        }
        if (wave == 0) {  // uniform: the four lane groups of a row store the same lse
          int row = row0 + 16 * ht + li;
          row = row < p.rows ? row : p.rows - 1;
          const float lse2 = xsum > 0.f ? m + __log2f(xsum) : -INFINITY;
          const int s = row / p.heads;
          const int h = row - s * p.heads;
          if (single) {
            if (p.lse != nullptr) p.lse[((int64_t)b * p.heads + h) * p.s_q + s] = lse2 * kLn2;
          } else {
            p.ws_lse[slot * p.rows + row] = lse2;
          }
        }
        lds_barrier();  // staging and merge words are read before their next use
      }
      continue;
    }
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      const float l = wave_sum_g(l_part[ht]);
      const float lx = wave_sum_g(l_exact[ht]);
      int row = row0 + 16 * ht + li;
      row = row < p.rows ? row : p.rows - 1;
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const float lse2 = lx > 0.f ? m_ref[ht] + __log2f(lx) : -INFINITY;
      const int s = row / p.heads;
      const int h = row - s * p.heads;
      // A single-split sequence writes its output directly (rounded once to the input dtype);
      // otherwise the split's partial goes to the workspace as scaled fp16 (each 128-dim chunk
      // held to 2^-11 of its amax), so the merged output's error stays within the 1e-2 bar.
      // (The reference's split kernel rounds its partials to the input dtype,
      // mla_decode.py:73-74,192; for bf16 that second rounding can move an output in [2, 4) by
      // up to 2^-7, past the bar.)
      const int64_t slot = slot0 + split;
      if (single) {  // uniform
        uint16_t* dst = p.out + (b * p.o_sb + s * p.o_ss + h * p.o_sh) + 4 * g;
#pragma unroll
        for (int dt = 0; dt < kDimTiles; ++dt) {  // one tile at a time (register pressure)
          const f32x4 v = o[dt][ht] * inv;
          *(i32x2*)(dst + 16 * dt) = i32x2{(int)pack2<DT>(v[0], v[1]), (int)pack2<DT>(v[2], v[3])};
          __builtin_amdgcn_sched_barrier(0);
        }
      } else if (p.part16) {  // uniform: 16-bit partials (the reference's own format)
        uint16_t* dst = p.ws_o + (slot * p.rows + row) * kDV + 4 * g;
#pragma unroll
        for (int dt = 0; dt < kDimTiles; ++dt) {
          const f32x4 v = o[dt][ht] * inv;
          *(i32x2*)(dst + 16 * dt) = i32x2{(int)pack2<DT>(v[0], v[1]), (int)pack2<DT>(v[2], v[3])};
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {  // scaled fp16: chunk c (tiles 8c .. 8c+7) of row li spans the four lane groups
        float am[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < kDimTiles; ++dt) am[dt >> 3] = fmaxf(am[dt >> 3], amax4(o[dt][ht]));
        int e[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float a = am[c] * inv;
          a = fmaxf(a, __shfl_xor(a, 16));
          a = fmaxf(a, __shfl_xor(a, 32));
          e[c] = part_exp(a);
        }
        uint16_t* dst = p.ws_o + (slot * p.rows + row) * kDV + 4 * g;
#pragma unroll
        for (int dt = 0; dt < kDimTiles; ++dt) {
          const f32x4 v = (o[dt][ht] * inv) * exp2i(e[dt >> 3]);
          *(i32x2*)(dst + 16 * dt) =
              i32x2{(int)pack2<MLA_DTYPE_F16>(v[0], v[1]), (int)pack2<MLA_DTYPE_F16>(v[2], v[3])};
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)  // the four lane groups store the same value (no divergence)
          p.ws_scale[(slot * p.rows + row) * 4 + c] = exp2i(-e[c]);
      }
      if (single) {
        if (p.lse != nullptr) p.lse[((int64_t)b * p.heads + h) * p.s_q + s] = lse2 * kLn2;
      } else {
        p.ws_lse[slot * p.rows + row] = lse2;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// wide kernel: 64 or 128 query rows per workgroup, PV split by output dims
// ---------------------------------------------------------------------------------------
// Four waves share a workgroup of R = 64*HT rows.  QK is split by rows: wave w owns rows
// 16*HT*w .. +16*HT (query fragments resident in VGPRs, S^T in VGPRs).  PV is split by output
// dims: wave w owns dims 128w .. 128w+127 of all R rows (8 x 4*HT accumulator tiles in AGPRs),
// so each wave reads only its quarter of V^T from LDS, and every V^T fragment feeds 4*HT
// MFMAs.  P^T crosses waves through LDS: each wave writes its row tiles' B fragments (one KiB
// each, lane-linear) and every wave reads all of them.  Iteration k of the stage loop runs QK
// of stage k, then the softmax of stage k next to PV of stage k-1 (whose P^T all waves wrote
// during iteration k-1), so a stage stays in LDS for two iterations.  LDS: a latent ring of 4
// 32-token stages (the stage of PV, the stage of QK, two in flight), a rope ring of 3 (rope is
// read by QK only), two P^T buffers.
//
// Stage layout.  Latent: 32 blocks of 1 KiB, block q*8 + s (row group q = rows 8q .. 8q+7,
// 128-byte segment s = dims 64s .. 64s+63); rope: 4 blocks, block q.  Inside a block, 16-byte
// chunk c8 of row r sits at slot 8*(r%8) + (c8 ^ stage_swz(r % 16)) (the layout of the
// one-ring kernel above, with the rope blocks moved to their own ring).
constexpr int kWideLat = 4;                  // latent stages resident
constexpr int kWideRope = 3;                 // rope stages resident
constexpr int kLatStageBytes = 32 * 1024;    // 32 token rows x 512 dims
constexpr int kRopeStageBytes = 4 * 1024;    // 32 token rows x 64 dims
constexpr int kWidePanel = 16 * 1024;        // tokens 16..31 of a latent stage

// FUSED: the latent and rope halves are one tensor (KParams::rope_fused), so a stage's rope rows
// are read from the latent row addresses + 1024 bytes (no second page lookup per stage), and
// each lane holds its page's 64-bit byte offset instead of its page id.
// sched: p.sched, preloaded (see mla_splitkv_kernel).  xcd_hb > 0: a 1-D grid of num_parts *
// xcd_hb workgroups (a multiple of 8), xcd_slots = its size / 8; XCD x runs a contiguous block
// of parts, the xcd_hb head blocks of a part in consecutive slots.  xcd_hb = 0: a (part, head
// block) grid.  Both are preloaded arguments too: the part index needs them before the record.
template <int DT, int HT, bool FUSED>
__global__ __launch_bounds__(256, 1) void mla_wide_kernel(const int32_t* __restrict__ sched, int xcd_hb, int xcd_slots,
                                                          KParams p) {
  constexpr int NW = 4;
  constexpr int RT = NW * HT;        // 16-row tiles per workgroup
  constexpr int R = 16 * RT;         // rows per workgroup
  constexpr int WDT = 8;             // 16-dim tiles per wave (128 dims)
  constexpr int DK = 4;              // LDS prefetch depth of the QK A fragments
  // Three placements in the stage loop that pay at 128 rows per workgroup and cost at 64 (C2 main
  // kernel 87.7 -> 86.5 us with all three; C5 50.5 -> 49.1 us with none of them at 64 rows):
  constexpr bool kMaskLate = HT == 2;   // QK results first read inside PV's first step
  constexpr bool kPtEarly = HT == 2;    // PV's first P^T fragments read at the end of QK
  constexpr bool kPrepEarly = HT == 2;  // stage k + 2's loads prepared at the end of iteration k - 1
  constexpr float kTau = ref_tau<DT>();
  constexpr int kPBytes = RT * 1024;
  __shared__ __attribute__((aligned(1024))) uint8_t lat_raw[kWideLat * kLatStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t rope_raw[kWideRope * kRopeStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t pt_raw[2 * kPBytes];
  __shared__ float inv_sh[R];   // 1 / row sum of every row, for the epilogue
  // "score above reference" words, one per stage modulo 4 (see the one-ring kernel)
  __shared__ int over_sh[4];
  uint8_t LDS_AS* const lat = (uint8_t LDS_AS*)lat_raw;
  uint8_t LDS_AS* const rope = (uint8_t LDS_AS*)rope_raw;
  uint8_t LDS_AS* const ptb = (uint8_t LDS_AS*)pt_raw;

  // Workgroups are handed to the 8 XCDs round-robin by linear id, each XCD starting its own
  // in order.  With a 1-D grid, id L is slot L / 8 of XCD L % 8, and XCD x owns the slots
  // x * G / 8 .. (x + 1) * G / 8 - 1 of the (part, head block) sequence, head blocks of a part
  // adjacent.  So the workgroups that read the same query rows (the splits and head blocks of
  // one sequence: consecutive parts) and the same pages (the head blocks of one part) run on
  // one XCD, together, and share its L2.
  int part, hb;
  if (xcd_hb > 0) {
    const int L = blockIdx.x;
    const int slot = (L & 7) * xcd_slots + (L >> 3);
    hb = xcd_hb == 1 ? 0 : slot % xcd_hb;
    part = xcd_hb == 1 ? slot : slot / xcd_hb;
  } else {
    part = blockIdx.x;
    hb = blockIdx.y;
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int li = lane & 15;
  const int rowb = hb * R;                 // the workgroup's first row (PV rows rowb .. +R)
  const int row0 = rowb + wave * 16 * HT;  // this wave's QK rows

  const int32_t* rec = sched + part * kSchedWords;
  int b = rec[0];
  int page = rec[1];
  const int end_b = rec[2];
  const int end_page = rec[3];
  int split = rec[4];

  // Per-lane LDS offsets of the fragments (recomputed from a fresh lane id, see the stage loop:
  // kept live across the loop they get spilled, and a reload before the loop makes the
  // compiler wait for every outstanding stage load inside it).
  // QK A operand, fragment (kk, tt), kk < 16: token row 16tt + li of latent chunk
  // sigma(kk, g) = 8*(kk/2) + 2g + kk%2, i.e. block (2tt + li/8)*8 + kk/2, chunk-in-block
  // 2g + kk%2: lane offset kl[kk%2] plus the immediate tt*16 KiB + (kk/2)*1 KiB.  kk = 16, 17:
  // the rope chunk 2g + kk%2 of rope block 2tt + li/8: kr[kk%2] + tt*2 KiB.
  // PV A operand (V^T), dim tile dt = 4s + d4 (segment s, tile d4 in it): the lane addresses
  // token row rv = 4g + li/4 (and row rv + 16 in the second panel), bytes 32*d4 + 8*(li%4) of
  // segment s; the swizzle flips only address bits 5-6 with d4, so the address is
  // (v_lane ^ 32*d4) + 1024*s.  Wave w's segments are 2w and 2w + 1.
  struct LaneOffsets {
    int kl0, kl1, kr0, kr1, v, pt;
  };
  // The chunks 2g and 2g + 1 of a row differ in bit 0, which the swizzle leaves in place, so
  // kl1 = kl0 ^ 16 and kr1 = kr0 ^ 16; kr0 is kl0 with its row-group bit (8 KiB) moved to 1 KiB.
  auto lane_offsets = [&](int ln) __attribute__((always_inline)) {
    const int gg = ln >> 4, ll = ln & 15;
    const int sw0 = (((ll & 7) << 3) + ((2 * gg) ^ stage_swz(ll))) << 4;
    const int r = 4 * gg + (ll >> 2);
    LaneOffsets o;
    o.kl0 = (ll >> 3) * 8192 + sw0;
    o.kl1 = o.kl0 ^ 16;
    o.kr0 = (ll >> 3) * 1024 + sw0;
    o.kr1 = o.kr0 ^ 16;
    o.v = (r >> 3) * 8192 + ((r & 7) << 7) + ((((ll >> 1) & 1) ^ stage_swz(r)) << 4) + ((ll & 1) << 3) + 2048 * wave;
    o.pt = 16 * ln;
    return o;
  };

  const int kv_st = (int)p.kv_st, kr_st = (int)p.kr_st;

#pragma unroll 1
  for (; b < p.batch; ++b, page = 0, split = 0) {
    if (!(b < end_b || (b == end_b && page < end_page))) break;
    // Segment prologue: the first 64 page ids, the query fragments, the length and the split
    // slots are requested back to back, in that order (nothing waits for the length before it
    // is requested last), so the segment starts after two memory round trips (these loads,
    // then its first stage) instead of one per dependent load.
    const bool paged = p.block_table != nullptr;

    int pbase = 0, bt_lane = 0;
    uint32_t pofs_lo = 0, pofs_hi = 0;  // FUSED: byte offset of page pbase + lane in the cache

    // page ids pbase .. pbase + 63 of the sequence, one per lane, clamped into the pool.  The
    // columns read stop at the table's width, not at the sequence's last page, so the load does
    // not wait for the length; only the ids of the sequence's own pages are ever used.  The
    // fused form turns them into byte offsets in finish_page_ids, after the other prologue
    // loads are issued.
    auto request_page_ids = [&](int first) __attribute__((always_inline)) {
      pbase = first;
      if (paged) {
        const int last = p.bt_width - 1;
        const int pi = pbase + fresh_lane() < last ? pbase + fresh_lane() : last;
        bt_lane = p.block_table[(int64_t)b * p.bt_stride + pi];
      }
    };
    auto finish_page_ids = [&]() __attribute__((always_inline)) {
      if (paged) {
        const int v = bt_lane;
        bt_lane = v < 0 ? 0 : (v >= p.num_blocks ? p.num_blocks - 1 : v);
        if constexpr (FUSED) {
          const uint64_t o = (uint64_t)(uint32_t)bt_lane * (uint32_t)p.kv_sp * 2;
          pofs_lo = (uint32_t)o;
          pofs_hi = (uint32_t)(o >> 32);
        }
      }
    };
    auto load_page_ids = [&](int first) __attribute__((always_inline)) {
      request_page_ids(first);
      finish_page_ids();
    };
    // ---- query fragments of this wave's rows (B operand of S^T = K Q^T), resident for the
    // segment; rows past the end re-load the last row (their results are never written).
    // The addresses come from a fresh lane id and an opaque copy of the head count: otherwise
    // their row-dependent parts (and the reciprocal behind the division by the head count) are
    // hoisted out of the segment loop and spilled, and each reload (on the in-order vmcnt)
    // waits for every load issued before it, a memory round trip apiece.
    request_page_ids(page);
    const int lq = fresh_lane();
    int heads_q = p.heads;
    asm volatile("" : "+s"(heads_q));
    i32x4 qf[HT][kKSteps];
    int qtok[HT];  // query token of each row tile's row
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      int row = row0 + 16 * ht + (lq & 15);
      row = row < p.rows ? row : p.rows - 1;
      const int s = row / heads_q;
      const int h = row - s * heads_q;
      qtok[ht] = s;
      const uint16_t* qn = p.q_nope + (b * p.q_sb + s * p.q_ss + h * p.q_sh) + 16 * (lq >> 4);
      const uint16_t* qr = p.q_rope + (b * p.qr_sb + s * p.qr_ss + h * p.qr_sh) + 16 * (lq >> 4);
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        const int d = 64 * (kk >> 1) + 8 * (kk & 1);  // dims 8*sigma(kk, g)
        qf[ht][kk] = *(const i32x4*)(d < kRopeOff ? qn + d : qr + (d - kRopeOff));
      }
    }
    // the length and the sequence's workspace slots (loaded here so that the epilogue does not
    // wait on them); awaiting the length also awaits everything above (vmcnt is in order),
    // which is in flight by then
    const int l_raw = p.seqlens[b];
    const int slot0 = p.splits[b];
    const bool single = (p.splits[b + 1] - slot0) == 1;
    const int L = bound_seq_len(p, l_raw, paged);
    finish_page_ids();
    const int np = pages_of(L);
    const int stop = (b == end_b) ? end_page : np;
    const int st_begin = 2 * page;
    const int st_end_seq = (L + kStageTok - 1) / kStageTok;
    const int st_end = (2 * stop < st_end_seq) ? 2 * stop : st_end_seq;
    const int nst = st_end > st_begin ? st_end - st_begin : 0;
    int lim[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) lim[ht] = L - (p.causal ? (p.s_q - 1 - qtok[ht]) : 0);
    const int lmin = L - (p.causal ? p.s_q - 1 : 0);  // every row sees tokens < lmin

    f32x4 o[WDT][RT];
    // row sums of this wave's QK rows: l_part over P as rounded for PV (normalises the
    // output), l_exact over the fp32 P (gives the lse)
    float m_ref[HT], l_part[HT], l_exact[HT];
    // The loads of one stage: wave w fetches row group w, 8 latent blocks and 1 rope block (one
    // global_load_lds_dwordx4 each, eight lanes per 128-byte line).  `prepare` does the scalar
    // work once (page lookup, 32 x 32 -> 64-bit page offset: page strides are below 2^32
    // elements, checked by the host); `issue_one(si, j)` issues load j, so the nine loads can
    // be spread between MFMAs (in a burst they hold the wave for ~900 cycles behind the CU's
    // load path; spread, ~10 each).  Rows past the sequence end re-read its last row.
    struct StageIssue {
      uint64_t nb, rb;  // latent and rope row bases of the stage (bytes, uniform)
      uint32_t on, orp; // per-lane byte offsets
      uint32_t lat_dst, rope_dst;  // LDS destinations (uniform)
    };
    // A stage past the segment (the loop's last iterations) is still issued, to the ring slot
    // that is free at that point, with every lane reading the segment's last row: the loads
    // cost a cache line, and the wait counts stay the same in every iteration.
    auto prepare = [&](int k) __attribute__((always_inline)) {
      const bool real = k < nst;
      const int st = st_begin + (real ? k : nst - 1);
      StageIssue si;
      const int tok = (st & 1) * kStageTok;
      const char* nb;
      const char* rb;
      if (paged && FUSED) {
        const int pidx = st >> 1;
        if (pidx - pbase >= 64) load_page_ids(pidx);  // uniform
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)pofs_lo, pidx - pbase);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)pofs_hi, pidx - pbase);
        nb = (const char*)p.kv_nope + ((((uint64_t)hi << 32) | lo) + (uint32_t)(tok * kv_st) * 2);
        rb = nb;  // unused: the rope load reads nb + 1024
      } else if (paged) {
        const int pidx = st >> 1;
        if (pidx - pbase >= 64) load_page_ids(pidx);  // uniform
        const uint32_t pg = (uint32_t)__builtin_amdgcn_readlane(bt_lane, pidx - pbase);
        nb = (const char*)p.kv_nope + ((uint64_t)pg * (uint32_t)p.kv_sp + (uint32_t)(tok * kv_st)) * 2;
        rb = (const char*)p.kv_rope + ((uint64_t)pg * (uint32_t)p.kr_sp + (uint32_t)(tok * kr_st)) * 2;
      } else {
        nb = (const char*)(p.kv_nope + ((int64_t)b * p.kv_sb + (int64_t)st * kStageTok * kv_st));
        rb = (const char*)(p.kv_rope + ((int64_t)b * p.kr_sb + (int64_t)st * kStageTok * kr_st));
      }
      const auto uni64 = [](const char* q) {
        const uint64_t v = (uint64_t)(uintptr_t)q;
        return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32)) << 32) |
               (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
      };
      si.nb = uni64(nb);
      si.rb = FUSED ? si.nb : uni64(rb);
      const int left = L - st * kStageTok;
      const int last_row = (left < kStageTok ? left : kStageTok) - 1;
      int row = 8 * wave + (lane >> 3);
      row = row < last_row && real ? row : last_row;
      const uint32_t cl = real ? (uint32_t)(((lane & 7) ^ stage_swz(((wave & 1) << 3) | (lane >> 3))) << 4) : 0u;
      si.on = (uint32_t)(row * kv_st) * 2 + cl;
      si.orp = FUSED ? si.on : (uint32_t)(row * kr_st) * 2 + cl;
      si.lat_dst = (uint32_t)__builtin_amdgcn_readfirstlane(
          (int)(uint32_t)(uintptr_t)(lat + (k % kWideLat) * kLatStageBytes + wave * 8 * 1024));
      si.rope_dst = (uint32_t)__builtin_amdgcn_readfirstlane(
          (int)(uint32_t)(uintptr_t)(rope + (k % kWideRope) * kRopeStageBytes + wave * 1024));
      return si;
    };
    auto issue_one = [&](const StageIssue& si, auto jtag) __attribute__((always_inline)) {
      constexpr int j = decltype(jtag)::value;
      if constexpr (j < 8) dma16_m0<j * 1024, 128 * j>(si.nb, si.on, si.lat_dst);
      else if constexpr (FUSED) dma16_m0<0, 1024>(si.nb, si.on, si.rope_dst);  // rope = latent row + 1024 B
      else dma16_m0<0>(si.rb, si.orp, si.rope_dst);
    };
    // load j (a constant once the loops around the call are unrolled)
    auto issue_j = [&](const StageIssue& si, int j) __attribute__((always_inline)) {
      switch (j) {
        case 0: issue_one(si, std::integral_constant<int, 0>{}); break;
        case 1: issue_one(si, std::integral_constant<int, 1>{}); break;
        case 2: issue_one(si, std::integral_constant<int, 2>{}); break;
        case 3: issue_one(si, std::integral_constant<int, 3>{}); break;
        case 4: issue_one(si, std::integral_constant<int, 4>{}); break;
        case 5: issue_one(si, std::integral_constant<int, 5>{}); break;
        case 6: issue_one(si, std::integral_constant<int, 6>{}); break;
        case 7: issue_one(si, std::integral_constant<int, 7>{}); break;
        default: issue_one(si, std::integral_constant<int, 8>{}); break;
      }
    };
    auto issue = [&](int k) __attribute__((always_inline)) {  // all nine at once
      const StageIssue si = prepare(k);
      issue_one(si, std::integral_constant<int, 0>{});
      issue_one(si, std::integral_constant<int, 1>{});
      issue_one(si, std::integral_constant<int, 2>{});
      issue_one(si, std::integral_constant<int, 3>{});
      issue_one(si, std::integral_constant<int, 4>{});
      issue_one(si, std::integral_constant<int, 5>{});
      issue_one(si, std::integral_constant<int, 6>{});
      issue_one(si, std::integral_constant<int, 7>{});
      issue_one(si, std::integral_constant<int, 8>{});
    };

    // One pass over the segment's stages; returns true (uniformly) when a first-stage-reference
    // pass saw a score above its reference by more than tau.
    //
    // Iteration k (1 <= k <= nst): wait for stage k, barrier, QK(k) with four of stage k+2's
    // loads between its MFMAs and, in its last steps, the reads of this wave's V^T fragments of
    // stage k-1; then PV(k-1) with the softmax of stage k and the other five loads woven into
    // it.  Iteration 0 (QK and softmax of stage 0) is peeled; the last iteration has no stage to
    // score and runs the same body with scores of -inf, so PV keeps a single site.
    auto run_pass = [&](auto mode_tag) __attribute__((always_inline)) -> bool {
      constexpr int MODE = decltype(mode_tag)::value;
      constexpr bool kPV = MODE != kPassRowMax;
      if constexpr (kPV) {
#pragma unroll
        for (int t = 0; t < WDT; ++t)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) o[t][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) l_part[ht] = l_exact[ht] = 0.f;
      }
      if constexpr (MODE != kPassFixedRef) {
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) m_ref[ht] = -INFINITY;
      }
      if constexpr (MODE == kPassFirstStageRef) {
        if (wave == 0) over_sh[lq & 3] = 0;  // uniform branch; ordered by the first barrier
      }
      // the first pass uses the page ids loaded in the prologue; a pass after an abort reloads
      // the window the segment starts in.  The compiler's wait for the ids (and for the query
      // fragments, before the first MFMA) counts only the loads issued after them.
      if (pbase != page) load_page_ids(page);  // uniform
      if (0 < nst) issue(0);
      if (1 < nst) issue(1);

      // V^T fragment t (t = 2*d4 + sl: segment 2w + sl, tile d4 in it) of stage kp
      auto v_frag = [&](const uint8_t LDS_AS* vb, int t) __attribute__((always_inline)) {
        const uint32_t x = (uint32_t)(32 * (t >> 1));
        const uint8_t LDS_AS* a = x ? (const uint8_t LDS_AS*)(uintptr_t)((uint32_t)(uintptr_t)vb ^ x) : vb;
        a += (t & 1) * 1024;
        const i16x4 lo16 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 LDS_AS*)a);
        const i16x4 hi16 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 LDS_AS*)(a + kWidePanel));
        const i32x2 lo2 = __builtin_bit_cast(i32x2, lo16);
        const i32x2 hi2 = __builtin_bit_cast(i32x2, hi16);
        return i32x4{lo2.x, lo2.y, hi2.x, hi2.y};
      };
      auto v_base = [&](int kp, const LaneOffsets& lo) __attribute__((always_inline)) {
        const uint8_t LDS_AS* vb = lat + (kp % kWideLat) * kLatStageBytes + lo.v;
        asm volatile("" : "+v"(vb));
        return vb;
      };
      // P^T fragment rt of stage kp (row tile rt's B operand of PV, one KiB, lane-linear)
      auto pt_frag = [&](int kp, const LaneOffsets& lo, int rt) __attribute__((always_inline)) {
        return *(const i32x4 LDS_AS*)(ptb + (kp & 1) * kPBytes + lo.pt + rt * 1024);
      };

      // S^T = K Q^T of stage k over 576 dims: two 16-token tiles x HT row tiles, fragment
      // n = 2*kk + tt, DK fragments in flight.  Loads 0..3 of `si` go out after steps 4, 12, 20
      // and 28; with `vt`, the V^T fragments of stage k-1 are read during the last 8 steps.
      // issue_tag: std::true_type to issue loads 0..3 of `si` between the MFMAs (the stage loop),
      // std::false_type for the peeled first iteration, which has no stage to issue
      // With `vt`, the first two P^T fragments of stage k-1 (PV's first two steps) are read in
      // the last steps too, and at 128 rows the QK results are left unsettled: PV's first step
      // issues eight MFMAs before the softmax reads them (see pv_softmax).
      auto qk = [&](int k, f32x4 (&acc)[HT][2], const LaneOffsets& lo, const StageIssue& si, auto issue_tag,
                    bool vt, i32x4 (&va)[WDT], i32x4 (&bq)[2]) __attribute__((always_inline)) {
        const uint8_t LDS_AS* lb = lat + (k % kWideLat) * kLatStageBytes;
        const uint8_t LDS_AS* rbs = rope + (k % kWideRope) * kRopeStageBytes;
        const uint8_t LDS_AS* kb0 = lb + lo.kl0;
        const uint8_t LDS_AS* kb1 = lb + lo.kl1;
        const uint8_t LDS_AS* rb0 = rbs + lo.kr0;
        const uint8_t LDS_AS* rb1 = rbs + lo.kr1;
        asm volatile("" : "+v"(kb0));
        asm volatile("" : "+v"(kb1));
        asm volatile("" : "+v"(rb0));
        asm volatile("" : "+v"(rb1));
        const uint8_t LDS_AS* vb = vt ? v_base(k - 1, lo) : lb;
#define MLA_WFRAG(N)                                                                                   \
  ((((N) >> 1) < 16)                                                                                   \
       ? *(const i32x4 LDS_AS*)((((N) >> 1) & 1 ? kb1 : kb0) + ((N) & 1) * kWidePanel + ((N) >> 2) * 1024) \
       : *(const i32x4 LDS_AS*)((((N) >> 1) & 1 ? rb1 : rb0) + ((N) & 1) * 2048))
        i32x4 kf[DK];
#pragma unroll
        for (int n = 0; n < DK; ++n) kf[n] = MLA_WFRAG(n);
#pragma unroll
        for (int n = 0; n < 2 * kKSteps; ++n) {
          const i32x4 a = kf[n % DK];
          if (n + DK < 2 * kKSteps) kf[n % DK] = MLA_WFRAG(n + DK);
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) {
            if (n < 2)
              mfma_qk_first<DT>(acc[ht][n & 1], a, qf[ht][n >> 1]);
            else
              mfma_qk<DT>(acc[ht][n & 1], a, qf[ht][n >> 1]);
          }
          if constexpr (decltype(issue_tag)::value) {
            if ((n & 7) == 4) issue_j(si, n >> 3);  // loads 0..3
          }
          if (n >= 2 * kKSteps - WDT && vt) va[n - (2 * kKSteps - WDT)] = v_frag(vb, n - (2 * kKSteps - WDT));
          if (kPtEarly && n >= 2 * kKSteps - 2 && vt) bq[n - (2 * kKSteps - 2)] = pt_frag(k - 1, lo, n - (2 * kKSteps - 2));
          __builtin_amdgcn_sched_barrier(0);
        }
#undef MLA_WFRAG
        const bool late = kMaskLate && vt;
        if (!late) qk_settle(acc[0][0]);
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
          if (ht > 0 || late) qk_touch(acc[ht][0]);
          qk_touch(acc[ht][1]);
        }
      };

      // mask tokens past each row's limit (uniform branch: the last stages only), then each
      // lane's largest scaled score per row tile
      auto mask_max = [&](int k, f32x4 (&acc)[HT][2], float (&lmx)[HT]) __attribute__((always_inline)) {
        const int st = st_begin + k;
        if (st * kStageTok + kStageTok > lmin) {
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) {
            int rel = lim[ht] - st * kStageTok - 4 * g;
            asm volatile("" : "+v"(rel));
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (16 * tt + r >= rel) acc[ht][tt][r] = -INFINITY;
          }
        }
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
          const float v = max3f(max3f(acc[ht][0][0], acc[ht][0][1], acc[ht][0][2]),
                                max3f(acc[ht][0][3], acc[ht][1][0], acc[ht][1][1]),
                                max3f(acc[ht][1][2], acc[ht][1][3], -INFINITY));
          lmx[ht] = v * p.scale_log2;
        }
      };

      // P^T = 2^(S^T * scale - m) of stage k as the B fragments of PV, row sums, fragments
      // published to P^T buffer k%2 (iteration 0 only; later stages go through pv_softmax)
      auto softmax_publish = [&](int k, const f32x4 (&acc)[HT][2]) __attribute__((always_inline)) {
        uint8_t LDS_AS* pw = ptb + (k & 1) * kPBytes + lane * 16;
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
          const float mu = m_ref[ht] == -INFINITY ? 0.f : m_ref[ht];
          float pv[2][4];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) pv[tt][r] = fast_exp2(acc[ht][tt][r] * p.scale_log2 - mu);
          const i32x4 pb = i32x4{(int)pack2<DT>(pv[0][0], pv[0][1]), (int)pack2<DT>(pv[0][2], pv[0][3]),
                                 (int)pack2<DT>(pv[1][0], pv[1][1]), (int)pack2<DT>(pv[1][2], pv[1][3])};
          l_part[ht] = packed_sum<DT>(pb, l_part[ht]);
          l_exact[ht] += ((pv[0][0] + pv[0][1]) + (pv[0][2] + pv[0][3])) +
                         ((pv[1][0] + pv[1][1]) + (pv[1][2] + pv[1][3]));
          *(i32x4 LDS_AS*)(pw + (wave * HT + ht) * 1024) = pb;
        }
      };

      // PV of stage kp (O^T += V^T P^T over its 32 tokens: this wave's 8 dim tiles x all RT row
      // tiles) with the softmax of stage kp + 1 and loads 4..8 of `si` woven in.  Step rt
      // streams P^T fragment rt (two steps ahead; fragments 0 and 1 come in `bq_in`, read at
      // the end of QK) against the 8 resident V^T fragments `va` (8 MFMAs), then computes two
      // P elements; the slicing is fixed in source order (one scheduling barrier per step),
      // which also bounds how many operands are live at once.  At 128 rows the QK results of
      // stage kp + 1 are first read after step 0's MFMAs (masking, the row maxima and the
      // `over` test), so the MFMA pipe goes from QK to PV without a gap; at 64 rows that placement
      // makes the register allocator spill, and mask_late_in_pv is false.
      auto pv_softmax = [&](int kp, f32x4 (&acc)[HT][2], const i32x4 (&va)[WDT], const i32x4 (&bq_in)[2],
                            const StageIssue& si, const LaneOffsets& lo,
                            bool& over) __attribute__((always_inline)) {
        uint8_t LDS_AS* pw = ptb + ((kp + 1) & 1) * kPBytes + lo.pt;
        float mu[HT];
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) mu[ht] = m_ref[ht] == -INFINITY ? 0.f : m_ref[ht];
        float pvv[HT][8];
        // softmax element e of the 8 * HT this lane owns: row tile e / 8, token tile (e / 4) % 2,
        // token 4g + e % 4 of it
        auto p_elem = [&](int e) __attribute__((always_inline)) {
          const int ht = e >> 3, tt = (e >> 2) & 1, r = e & 3;
          pvv[ht][e & 7] = fast_exp2(acc[ht][tt][r] * p.scale_log2 - mu[ht]);
        };
        auto p_finish = [&](int ht) __attribute__((always_inline)) {
          const float* v = pvv[ht];
          const i32x4 pb = i32x4{(int)pack2<DT>(v[0], v[1]), (int)pack2<DT>(v[2], v[3]),
                                 (int)pack2<DT>(v[4], v[5]), (int)pack2<DT>(v[6], v[7])};
          l_part[ht] = packed_sum<DT>(pb, l_part[ht]);
          l_exact[ht] += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
          *(i32x4 LDS_AS*)(pw + (wave * HT + ht) * 1024) = pb;
        };
        constexpr int kPer = (8 * HT + RT - 1) / RT;  // P elements per step: 2
        i32x4 bq[2] = {bq_in[0], bq_in[1]};
        i32x4 b_last = bq[0];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const i32x4 bcur = bq[rt & 1];
          if (rt + 2 < RT) bq[rt & 1] = pt_frag(kp, lo, rt + 2);
#pragma unroll
          for (int t = 0; t < WDT; ++t) o[t][rt] = mfma32<DT>(va[t], bcur, o[t][rt]);
          if (kMaskLate && rt == 0) {
            // eight MFMAs and 12 more wait states since the last QK MFMA: its results are
            // readable (the documented need is at most 19 wait states)
            qk_settle_after_mfmas(acc);
            float lmx[HT];
            mask_max(kp + 1, acc, lmx);
            if constexpr (MODE == kPassFirstStageRef) {
#pragma unroll
              for (int ht = 0; ht < HT; ++ht) over |= lmx[ht] > m_ref[ht] + kTau;
            }
          }
#pragma unroll
          for (int q = 0; q < kPer; ++q) {
            const int e = rt * kPer + q;
            if (e < 8 * HT) {
              p_elem(e);
              if ((e & 7) == 7) p_finish(e >> 3);
            }
          }
          // loads 4..8 after steps (2i + 1) * RT / 10
#pragma unroll
          for (int i = 0; i < 5; ++i)
            if (rt == (2 * i + 1) * RT / 10) issue_j(si, 4 + i);
          __builtin_amdgcn_sched_barrier(0);
          b_last = bcur;
        }
        // the last MFMAs still read their operands for several passes after they issue
        i32x4 v7 = va[WDT - 1];
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(v7), "+v"(b_last));
      };

      bool abort = false;
      if (nst > 0) {  // ---- iteration 0: QK and softmax of stage 0, all loads of stage 2
        if (1 < nst) wait_vmcnt<9>();  // stage 0 landed; stage 1 may stay in flight
        else wait_vmcnt<0>();
        wait_lgkm0();
        lds_barrier();
        if (2 < nst) issue(2);
        const int ln0 = fresh_lane();
        const LaneOffsets lo = lane_offsets(ln0);
        f32x4 acc[HT][2];
        i32x4 va_unused[WDT], bq_unused[2];
        qk(0, acc, lo, StageIssue{}, std::false_type{}, false, va_unused, bq_unused);
        float lmx[HT];
        mask_max(0, acc, lmx);
        if constexpr (MODE == kPassRowMax) {
#pragma unroll
          for (int ht = 0; ht < HT; ++ht) m_ref[ht] = fmaxf(m_ref[ht], lmx[ht]);
        } else {
          if constexpr (MODE == kPassFirstStageRef) {
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) m_ref[ht] = wave_max_g(lmx[ht]);
          }
          softmax_publish(0, acc);
        }
      }
      // ---- k = 1 .. nst
      const int lnp = fresh_lane();
      const LaneOffsets lo_pass = lane_offsets(lnp);
      const int kend = kPV ? nst + 1 : nst;
      // the loads of stage k + 2, prepared at the end of iteration k - 1 (while the wave waits
      // for its P^T stores before the barrier) rather than between the barrier and QK
      StageIssue si;
      if constexpr (kPrepEarly) si = prepare(3);
#pragma unroll 1
      for (int k = 1; k < kend; ++k) {
        const bool has_qk = k < nst;  // uniform
        if (has_qk) {
          if (k + 1 < nst) wait_vmcnt<9>();  // stage k landed; stage k+1 may stay in flight
          else wait_vmcnt<0>();
        }
        wait_lgkm0();  // this wave's P^T and flag stores of iteration k-1 have landed
        lds_barrier();
        // the flag word of stage k-1 (stage 0 sets the reference and never flags), consumed
        // after QK; wave 0 clears the word of stage k-2, read by every wave in iteration k-1
        int flag_word = 0;
        if constexpr (MODE == kPassFirstStageRef) {
          flag_word = over_sh[(k - 1) & 3];
          if (k >= 3 && wave == 0) over_sh[(k - 2) & 3] = 0;
        }
        if constexpr (!kPrepEarly) si = prepare(k + 2);  // past the segment: dummy loads
        // 64-row form: from a fresh lane id per iteration (kept live across the loop they
        // spill); 128-row form: once per pass (no spill there, 27 fewer VALU per stage)
        const LaneOffsets lo = HT == 1 ? lane_offsets(fresh_lane()) : lo_pass;
        f32x4 acc[HT][2];
        i32x4 va[WDT];
        i32x4 bq[2];
        if (has_qk) {
          qk(k, acc, lo, si, std::true_type{}, kPV, va, bq);
          if constexpr (kPV && !kPtEarly) {
            bq[0] = pt_frag(k - 1, lo, 0);
            bq[1] = pt_frag(k - 1, lo, 1);
          }
        } else {
          // scores of -inf, set inside this branch (as constants the compiler would hoist the
          // sixteen moves out of it, into every iteration)
#pragma unroll
          for (int ht = 0; ht < HT; ++ht)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[ht][tt][r] = neg_inf_here();
          if constexpr (kPV) {
            const uint8_t LDS_AS* vb = v_base(k - 1, lo);
#pragma unroll
            for (int t = 0; t < WDT; ++t) va[t] = v_frag(vb, t);
            bq[0] = pt_frag(k - 1, lo, 0);
            bq[1] = pt_frag(k - 1, lo, 1);
          }
        }
        if constexpr (MODE == kPassFirstStageRef) {
          if (flag_word != 0) {  // uniform: every wave read the same word after the same barrier
            abort = true;
            break;
          }
        }
        bool over = false;
        if constexpr (!kPV || !kMaskLate) {
          float lmx[HT];
          mask_max(k, acc, lmx);
          if constexpr (MODE == kPassRowMax) {
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) m_ref[ht] = fmaxf(m_ref[ht], lmx[ht]);
          } else if constexpr (MODE == kPassFirstStageRef) {
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) over |= lmx[ht] > m_ref[ht] + kTau;
          }
        }
        if constexpr (kPV) {
          pv_softmax(k - 1, acc, va, bq, si, lo, over);
        } else {
#pragma unroll
          for (int j = 4; j < 9; ++j) issue_j(si, j);
        }
        if constexpr (MODE == kPassFirstStageRef) {
          if (__builtin_amdgcn_ballot_w64(over) != 0) over_sh[k & 3] = 1;  // uniform branch
        }
        if constexpr (kPrepEarly) si = prepare(k + 3);  // past the segment: dummy loads (see prepare)
      }
      wait_vmcnt<0>();  // an abandoned pass may leave stage loads in flight
      wait_lgkm0();
      lds_barrier();    // every wave is done with the rings and P^T buffers
      return abort;
    };

    if (run_pass(std::integral_constant<int, kPassFirstStageRef>{})) {
      run_pass(std::integral_constant<int, kPassRowMax>{});
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) m_ref[ht] = wave_max_g(m_ref[ht]);
      run_pass(std::integral_constant<int, kPassFixedRef>{});
    }

    // ---- epilogue.  The QK-owning wave finishes its rows' sums, writes their lse and
    // publishes 1 / (row sum); then every wave normalises its dims of all R rows.  Branch-free
    // apart from uniform branches; padding rows (past the last row) compute and store the last
    // row's values.
    const int64_t slot = slot0 + split;
    // A fresh lane id and an opaque copy of the head count: the (row -> token, head) division below
    // otherwise reuses a constant formed at kernel start, spilled, whose reload in each row
    // tile waits (in-order vmcnt) for every store issued before it.
    const int lane_e = fresh_lane();
    int heads_e = p.heads;
    asm volatile("" : "+v"(heads_e));
    const int li_e = lane_e & 15, g_e = lane_e >> 4;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      const float l = wave_sum_g(l_part[ht]);
      const float lx = wave_sum_g(l_exact[ht]);
      int row = row0 + 16 * ht + li_e;
      row = row < p.rows ? row : p.rows - 1;
      inv_sh[wave * 16 * HT + 16 * ht + li_e] = l > 0.f ? 1.f / l : 0.f;  // four lane groups, one value
      const float lse2 = lx > 0.f ? m_ref[ht] + __log2f(lx) : -INFINITY;
      const int s = row / heads_e;
      const int h = row - s * heads_e;
      if (single) {
        if (p.lse != nullptr) p.lse[((int64_t)b * heads_e + h) * p.s_q + s] = lse2 * kLn2;
      } else {
        p.ws_lse[slot * p.rows + row] = lse2;
      }
    }
    wait_lgkm0();
    lds_barrier();
    // The wave's 128 dims of all R rows go out through its 32 KiB quarter of the latent ring
    // (free after the pass): packed to 16 bits and written there in rows of 256 bytes, then
    // read back so that each global store writes four whole row slices, 16 bytes per lane and
    // eight full cache lines per instruction.  Stored straight from the fragment layout, each
    // instruction wrote 32-byte pieces of 16 lines, and the store path took ~60 cycles per
    // instruction: ~2000 per row tile.  In the staging rows, 32-byte chunk c of row r sits at
    // chunk c ^ (r % 8), and its 8-byte piece j (dims 4j .. 4j+3 of the chunk) at piece
    // j ^ (2 * ((r / 8) % 2)): a fragment write (8 bytes from each of 16 rows, two lane groups
    // per half-wave) then covers all 64 banks in each half-wave, rows 0-7 of the tile in the
    // first 16 bytes of their chunks and rows 8-15 in the second.
    uint8_t LDS_AS* const stg = lat + wave * (32 * 1024);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float inv = inv_sh[16 * rt + li_e];
      const int r = 16 * rt + li_e;  // row of the workgroup
      // bits 3-7 of the row's LDS address are zero, so the chunk and piece permutations are
      // one XOR
      const uint32_t srow = (uint32_t)(uintptr_t)(stg + r * 256 + 8 * g_e) ^
                            (uint32_t)(((r & 7) << 5) | (((r >> 3) & 1) << 4));
      // fragment t holds dims 64*(t%2) + 16*(t/2) + 4g .. +3 of the slice: chunk 4*(t%2) + t/2
      auto put = [&](int t, const i32x2 v) __attribute__((always_inline)) {
        *(i32x2 LDS_AS*)(uintptr_t)(srow ^ (uint32_t)((4 * (t & 1) + (t >> 1)) << 5)) = v;
      };
      if (single || p.part16) {  // uniform
#pragma unroll
        for (int t = 0; t < WDT; ++t) {
          const f32x4 v = o[t][rt] * inv;
          put(t, i32x2{(int)pack2<DT>(v[0], v[1]), (int)pack2<DT>(v[2], v[3])});
        }
      } else {  // scaled fp16: the wave's chunk of row r spans the four lane groups
        float am = 0.f;
#pragma unroll
        for (int t = 0; t < WDT; ++t) am = fmaxf(am, amax4(o[t][rt]));
        am *= inv;
        am = xor32_max(xor16_max(am));
        const int e = part_exp(am);
        const float f = inv * exp2i(e);  // o * (inv * 2^e) rounds exactly as (o * inv) * 2^e
#pragma unroll
        for (int t = 0; t < WDT; ++t) {
          const f32x4 v = o[t][rt] * f;
          put(t, i32x2{(int)pack2<MLA_DTYPE_F16>(v[0], v[1]), (int)pack2<MLA_DTYPE_F16>(v[2], v[3])});
        }
        int row = rowb + r;
        row = row < p.rows ? row : p.rows - 1;
        p.ws_scale[(slot * p.rows + row) * 4 + wave] = exp2i(-e);  // four lane groups, one value
      }
    }
    // rows 4j .. 4j+3: lane l moves bytes 16*(l%16) .. +15 of row 4j + l/16 (this wave's own
    // staging rows: no barrier, LDS runs one wave's accesses in order)
    {
      const int q = lane_e & 15;
      const int r0 = lane_e >> 4;
      auto staged = [&](int j) __attribute__((always_inline)) {
        const int r = 4 * j + r0;
        return *(const i32x4 LDS_AS*)(stg + r * 256 + ((((q >> 1) ^ (r & 7)) << 5) | (((q ^ (r >> 3)) & 1) << 4)));
      };
      // uniform: the workgroup's rows are one run of rows in the destination (no padding rows,
      // one query token), so row r is at a fixed stride from row 0
      const bool linear = rowb + R <= p.rows && (!single || (rowb % heads_e) + R <= heads_e);
      if (linear) {
        int64_t stride;
        uint16_t* dst;
        if (single) {
          const int s = rowb / heads_e;
          const int h = rowb - s * heads_e + r0;
          dst = p.out + (b * p.o_sb + s * p.o_ss + h * p.o_sh) + 128 * wave + 8 * q;
          stride = 4 * p.o_sh;
        } else {
          dst = p.ws_o + (slot * p.rows + rowb + r0) * kDV + 128 * wave + 8 * q;
          stride = 4 * kDV;
        }
#pragma unroll 4
        for (int j = 0; j < R / 4; ++j) *(i32x4*)(dst + j * stride) = staged(j);
      } else {
#pragma unroll 2
        for (int j = 0; j < R / 4; ++j) {
          int row = rowb + 4 * j + r0;
          row = row < p.rows ? row : p.rows - 1;  // padding rows repeat the last row's values
          uint16_t* dst;
          if (single) {  // uniform
            const int s = row / heads_e;
            const int h = row - s * heads_e;
            dst = p.out + (b * p.o_sb + s * p.o_ss + h * p.o_sh);
          } else {
            dst = p.ws_o + (slot * p.rows + row) * kDV;
          }
          *(i32x4*)(dst + 128 * wave + 8 * q) = staged(j);
        }
      }
    }
    wait_lgkm0();
    lds_barrier();  // the staging reads are done before the next segment's loads refill the ring
    // inv_sh is rewritten only after the next segment's barriers
  }
}

// The dense wave-split decode (up to 16 query rows: the batch-1 and small-head shapes) is
// instantiated and launched in its own translation unit, mla_decode_ws.hip, which the build
// compiles with LLVM's iterative ILP machine scheduler: that schedule of the kernel's stage
// loop measured 1.5% faster at 16 heads over ragged long sequences and 6.5% faster at batch
// 1, and the same scheduler made the wide kernel slower, so it is not used for this file.
template <int DT>
hipError_t launch_ws_dense(const KParams& kp, int head_blocks, hipStream_t st);

#ifdef MLA_WS_TU
template <int DT>
hipError_t launch_ws_dense(const KParams& kp, int head_blocks, hipStream_t st) {
  hipLaunchKernelGGL((mla_splitkv_kernel<DT, 4, 1, 1, true, false, false>), dim3(kp.num_parts, head_blocks),
                     dim3(4 * 64), 0, st, kp.sched, kp);
  return hipGetLastError();
}
template hipError_t launch_ws_dense<MLA_DTYPE_BF16>(const KParams&, int, hipStream_t);
template hipError_t launch_ws_dense<MLA_DTYPE_F16>(const KParams&, int, hipStream_t);
}  // namespace mla
#else

// ---------------------------------------------------------------------------------------
// paged KV-cache append: one wave per sequence (its length is read once, before its rows are
// written, and advanced after them); lanes 0..63 copy the 512 latent dims and lanes 0..7
// the 64 rope dims of each new row, 16 bytes per lane
// ---------------------------------------------------------------------------------------
struct AppendParams {
  const uint16_t* kv_new;
  int64_t n_sb, n_st;
  uint16_t* kv_nope;
  uint16_t* kv_rope;
  int64_t kv_sp, kv_st, kr_sp, kr_st;
  const int32_t* block_table;
  int32_t bt_stride, max_pages, num_blocks, batch, n_new;
  int32_t* seqlens;
  int32_t* status;
  // fp8 cache (kv8 != 0): kv_nope holds e4m3 codes (strides in bytes), kv_scale the scales
  int32_t kv8;
  float* kv_scale;
  int64_t ks_sp, ks_sb;
};

// The power-of-two exponent k of a 128-dim block's scale from its bf16 amax (bit pattern
// `bits`): the smallest k with amax <= 448 * 2^k (448 = 1.75 * 2^8, mantissa 0x60), clamped
// to [-126, 127]; amax = 0 gives 0.
__device__ __forceinline__ int fp8_block_exp(uint32_t bits) {
  const int ef = (int)((bits >> 7) & 0xFF);
  const int mant = (int)(bits & 0x7F);
  int k = ef - 127 - 8 + (mant > 0x60 ? 1 : 0);
  if (ef == 0) k = -126;
  if (bits == 0) k = 0;
  return k < -126 ? -126 : (k > 127 ? 127 : k);
}

__global__ __launch_bounds__(256) void mla_kv_append_kernel(AppendParams a) {
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= a.batch) return;  // whole waves only
  const int L = a.seqlens[b];
  bool ok = L >= 0;
  for (int t = 0; t < a.n_new; ++t) {
    const int pos = L + t;
    const int pi = pos >> 6;
    if (pi >= a.max_pages) {
      ok = false;
    } else {
      const int pg = a.block_table[(int64_t)b * a.bt_stride + pi];
      ok = ok && pg >= 0 && pg < a.num_blocks;
    }
  }
  if (!ok) {
    if (lane == 0 && a.status != nullptr) a.status[0] = 1;
    return;
  }
  for (int t = 0; t < a.n_new; ++t) {
    const int pos = L + t;
    const int pg = a.block_table[(int64_t)b * a.bt_stride + (pos >> 6)];
    const int row = pos & 63;
    const uint16_t* src = a.kv_new + b * a.n_sb + t * a.n_st;
    const i32x4 v = *(const i32x4*)(src + 8 * lane);
    if (a.kv8) {  // uniform
      // lane l holds dims 8l .. 8l+7; block j (dims 128j ..) is the lane group of 16
      float x[8];
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int w = v[i];
        x[2 * i] = __uint_as_float((uint32_t)w << 16);
        x[2 * i + 1] = __uint_as_float((uint32_t)w & 0xFFFF0000u);
        amax = fmaxf(amax, fmaxf(fabsf(x[2 * i]), fabsf(x[2 * i + 1])));
      }
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 16));
      const int k = fp8_block_exp(__float_as_uint(amax) >> 16);  // amax is a bf16 value
      int lo = 0, hi = 0;
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_ldexpf(x[0], -k), __builtin_ldexpf(x[1], -k), lo, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_ldexpf(x[2], -k), __builtin_ldexpf(x[3], -k), lo, true);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_ldexpf(x[4], -k), __builtin_ldexpf(x[5], -k), hi, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_ldexpf(x[6], -k), __builtin_ldexpf(x[7], -k), hi, true);
      uint8_t* dst = (uint8_t*)a.kv_nope + (int64_t)pg * a.kv_sp + (int64_t)row * a.kv_st + 8 * lane;
      *(i32x2*)dst = i32x2{lo, hi};
      if ((lane & 15) == 0)
        a.kv_scale[(int64_t)pg * a.ks_sp + (int64_t)(lane >> 4) * a.ks_sb + row] =
            __uint_as_float((uint32_t)(k + 127) << 23);
    } else {
      *(i32x4*)(a.kv_nope + (int64_t)pg * a.kv_sp + (int64_t)row * a.kv_st + 8 * lane) = v;
    }
    if (lane < 8) {
      const i32x4 r = *(const i32x4*)(src + kRopeOff + 8 * lane);
      *(i32x4*)(a.kv_rope + (int64_t)pg * a.kr_sp + (int64_t)row * a.kr_st + 8 * lane) = r;
    }
  }
  if (lane == 0) a.seqlens[b] = L + a.n_new;
}

// ---------------------------------------------------------------------------------------
// combine: LSE-weighted merge of the splits of each (sequence, row)
// ---------------------------------------------------------------------------------------
// Eight consecutive partial values of one row, widened to fp32: the fp32 rows of
// mla_merge_partials, or the 16-bit rows of the decode workspace and of mla_launch.
template <int DT>
__device__ __forceinline__ void load8(const float* src, float (&x)[8]) {
  const f32x4 a = *(const f32x4*)src;
  const f32x4 c = *(const f32x4*)(src + 4);
  x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
  x[4] = c[0]; x[5] = c[1]; x[6] = c[2]; x[7] = c[3];
}
template <int DT>
__device__ __forceinline__ void cvt8(const i32x4 v, float (&x)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (DT == MLA_DTYPE_BF16) {
      x[2 * j] = __builtin_bit_cast(float, (uint32_t)v[j] << 16);
      x[2 * j + 1] = __builtin_bit_cast(float, (uint32_t)v[j] & 0xffff0000u);
    } else {
      // copied to a scalar first: __builtin_bit_cast applied to the vector element itself
      // compiled to a read of element 0 for every j
      const int w = v[j];
      const f16x2 h = __builtin_bit_cast(f16x2, w);
      x[2 * j] = (float)h[0];
      x[2 * j + 1] = (float)h[1];
    }
  }
}
template <int DT>
__device__ __forceinline__ void load8(const uint16_t* src, float (&x)[8]) {
  cvt8<DT>(*(const i32x4*)src, x);
}

// Merge of one row's split partials by one wave; lane l owns columns 8l .. 8l+7.  Split weights
// are exp2(lse_k - lse) with lse the log2-sum-exp2 over the row's n splits, staged through the
// wave's 64-float LDS slot so every lane reads them; the partial rows are read four splits at a
// time (independent loads).  Returns lse (log2; -inf when no split saw a key, acc then zero).
// SCALED: fp16 rows whose 128-dim chunk c carries the factor ws_scale[(slot, row) * 4 + c]
// (lane l's chunk is l / 16), folded into the split weight.  The fused absorb prologue repeats
// this arithmetic operation for operation.
template <int DT, typename PT, bool SCALED>
__device__ __forceinline__ float merge_splits_wave(const PT* __restrict__ ws_o, const float* __restrict__ ws_scale,
                                                   const float* __restrict__ ws_lse, int base, int n, int rows,
                                                   int row, int lane, float* w_sh, float (&acc)[8]) {
  constexpr int LDT = SCALED ? MLA_DTYPE_F16 : DT;  // element type of the partial rows
  float mx = -INFINITY;
  for (int k = lane; k < n; k += 64) mx = fmaxf(mx, ws_lse[(int64_t)(base + k) * rows + row]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float sum = 0.f;
  if (mx != -INFINITY)
    for (int k = lane; k < n; k += 64) sum += fast_exp2(ws_lse[(int64_t)(base + k) * rows + row] - mx);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  const float lse2 = sum > 0.f ? mx + __log2f(sum) : -INFINITY;

#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  const PT* src0 = ws_o + ((int64_t)base * rows + row) * kDV + lane * 8;
  const int64_t split_stride = (int64_t)rows * kDV;
  const float* sc0 = SCALED ? ws_scale + ((int64_t)base * rows + row) * 4 + (lane >> 4) : nullptr;
  const int64_t sc_stride = (int64_t)rows * 4;
  for (int k0 = 0; k0 < n; k0 += 64) {
    const int k = k0 + lane;
    float w = 0.f;
    if (k < n && lse2 != -INFINITY) w = fast_exp2(ws_lse[(int64_t)(base + k) * rows + row] - lse2);
    w_sh[lane] = w;
    __builtin_amdgcn_wave_barrier();
    const int kn = n - k0 < 64 ? n - k0 : 64;
    int kk = 0;
    for (; kk + 4 <= kn; kk += 4) {
      float x[4][8], us[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        load8<LDT>(src0 + (k0 + kk + u) * split_stride, x[u]);
        us[u] = SCALED ? sc0[(k0 + kk + u) * sc_stride] : 1.f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float wk = w_sh[kk + u] * us[u];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += wk * x[u][j];
      }
    }
    for (; kk < kn; ++kk) {
      float x[8];
      load8<LDT>(src0 + (k0 + kk) * split_stride, x);
      const float wk = w_sh[kk] * (SCALED ? sc0[(k0 + kk) * sc_stride] : 1.f);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += wk * x[j];
    }
    __builtin_amdgcn_wave_barrier();
  }
  return lse2;
}

// merge_splits_wave for a row of at most kFewSplits 16-bit partials, in one memory round trip:
// the lse values, partial rows and chunk scales of all its splits are requested together (the
// partials do not depend on the weights), then merged with merge_splits_wave's arithmetic
// operation for operation, so the result is bit-identical: the same max, the same sum in the
// order of its xor butterfly (splits k >= n contribute zeros, which leave every partial sum
// unchanged), the same weights and the same fma chain in split order.
constexpr int kFewSplits = 8;
template <int DT, bool SCALED>
__device__ __forceinline__ float merge_few_splits(const uint16_t* __restrict__ ws_o, const float* __restrict__ ws_scale,
                                                  const float* __restrict__ ws_lse, int base, int n, int rows,
                                                  int row, int lane, float (&acc)[8]) {
  constexpr int LDT = SCALED ? MLA_DTYPE_F16 : DT;
  const uint16_t* src0 = ws_o + ((int64_t)base * rows + row) * kDV + lane * 8;
  const int64_t split_stride = (int64_t)rows * kDV;
  const float* sc0 = SCALED ? ws_scale + ((int64_t)base * rows + row) * 4 + (lane >> 4) : nullptr;
  const int64_t sc_stride = (int64_t)rows * 4;
  float l[kFewSplits], us[kFewSplits];
  i32x4 raw[kFewSplits];
#pragma unroll
  for (int k = 0; k < kFewSplits; ++k) {
    l[k] = -INFINITY;
    us[k] = 1.f;
    raw[k] = i32x4{0, 0, 0, 0};
    if (k < n) {  // uniform
      l[k] = ws_lse[(int64_t)(base + k) * rows + row];
      raw[k] = *(const i32x4*)(src0 + k * split_stride);
      if constexpr (SCALED) us[k] = sc0[k * sc_stride];
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kFewSplits; ++k) mx = fmaxf(mx, l[k]);
  float e[kFewSplits];
#pragma unroll
  for (int k = 0; k < kFewSplits; ++k) e[k] = (mx != -INFINITY && k < n) ? fast_exp2(l[k] - mx) : 0.f;
  // the butterfly's association: offsets 32, 16 and 8 add zeros, then 4, 2, 1
  const float sum = ((e[0] + e[4]) + (e[2] + e[6])) + ((e[1] + e[5]) + (e[3] + e[7]));
  const float lse2 = sum > 0.f ? mx + __log2f(sum) : -INFINITY;
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
#pragma unroll
  for (int k = 0; k < kFewSplits; ++k) {
    if (k < n) {  // uniform
      float x[8];
      cvt8<LDT>(raw[k], x);
      const float w = lse2 != -INFINITY ? fast_exp2(l[k] - lse2) : 0.f;
      const float wk = w * us[k];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += wk * x[j];
    }
  }
  return lse2;
}

// merge_splits_wave for a row of at most kDeepSplits 16-bit partials, by four waves that each
// take one 128-dim quarter q of the row (lane l: dims 128 q + 2 l, +1), so a long merge runs on
// four CUs instead of one.  A wave keeps kQueue quarter rows in flight in a register queue: the
// loop, unrolled by kQueue, consumes split k from queue slot k % kQueue and reloads that slot
// with split k + kQueue (an index past the last split is clamped to it), so consuming a slot
// waits only for that slot's load.  The loop is issue-bound (one wave per SIMD; the queue depth
// does not matter between 16 and 32), so a block whose splits are all live runs without the
// per-split zeroing of surplus rows that the last block needs.  The lse of all splits (lane l
// holds splits l, l + 64, ..) and the quarter's chunk scale come first; the weight of split k
// times that scale is formed once, into kw[k] (0 past the last split).  Arithmetic per output
// element is merge_splits_wave's operation for operation (the same per-lane order of the max
// and the sum, the same butterfly, the same product w * s and fma chain in split order): the
// result is bit-identical.  (An LDS-DMA ring in place of the queue was no faster.)
constexpr int kDeepSplits = 256;
constexpr int kDeepMaxRows = 16384;  // kDeepSplits * kDeepMaxRows KiB = 2^32 bytes
constexpr int kQueue = 32;
constexpr int kDeepLds = (kDeepSplits + kQueue) * 4;  // kw
template <int DT, bool SCALED>
__device__ __forceinline__ float merge_many_splits(const uint16_t* __restrict__ ws_o, const float* __restrict__ ws_scale,
                                                   const float* __restrict__ ws_lse, int base, int n, int rows,
                                                   int row, int q, int lane, char* smem, float (&acc)[2]) {
  static_assert(kDeepSplits % 64 == 0 && kQueue <= 63 && kQueue % 4 == 0 && kQueue <= 64, "queue shape");
  constexpr int LDT = SCALED ? MLA_DTYPE_F16 : DT;
  constexpr int kL = kDeepSplits / 64;
  float* kw = (float*)smem;
  // split k's quarter row: a uniform base plus the lane's 4 bytes.  Offsets are 32-bit: the host
  // takes this path only for rows <= kDeepMaxRows, so the last split's offset, at most
  // (kDeepSplits - 1) * rows KiB, stays below 2^32 (a surplus load's offset may wrap, to an
  // earlier split of the same row, and is consumed as zeros)
  const char* row0 = (const char*)(ws_o + ((int64_t)base * rows + row) * kDV + 128 * q);
  const uint32_t split_bytes = (uint32_t)rows * kDV * 2;
  const float* lp = ws_lse + (int64_t)base * rows + row;
  const int last = n - 1;
  const uint32_t last_off = (uint32_t)last * split_bytes;
  uint32_t next_off = 0;  // the next split to load, clamped to the last
  auto load_next = [&]() __attribute__((always_inline)) {
    const uint32_t v = *(const uint32_t*)(row0 + next_off + lane * 4);
    next_off = next_off + split_bytes < last_off ? next_off + split_bytes : last_off;
    return v;
  };

  float lv[kL], sc[kL];
#pragma unroll
  for (int c = 0; c < kL; ++c) {
    const int k = c * 64 + lane;
    const int kc = k < last ? k : last;
    const float l = lp[(int64_t)kc * rows];
    lv[c] = k < n ? l : -INFINITY;
    if constexpr (SCALED) sc[c] = ws_scale[((int64_t)(base + kc) * rows + row) * 4 + q];
  }
  uint32_t qv[kQueue];
#pragma unroll
  for (int u = 0; u < kQueue; ++u) qv[u] = load_next();

  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < kL; ++c)
    if (c * 64 + lane < n) mx = fmaxf(mx, lv[c]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float sum = 0.f;
  if (mx != -INFINITY)
#pragma unroll
    for (int c = 0; c < kL; ++c)
      if (c * 64 + lane < n) sum += fast_exp2(lv[c] - mx);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  const float lse2 = sum > 0.f ? mx + __log2f(sum) : -INFINITY;
#pragma unroll
  for (int c = 0; c < kL; ++c) {
    const int k = c * 64 + lane;
    float w = 0.f;
    if (k < n && lse2 != -INFINITY) w = fast_exp2(lv[c] - lse2);
    kw[k] = SCALED ? w * sc[c] : w;
  }
  if (lane < kQueue) kw[kDeepSplits + lane] = 0.f;
  __builtin_amdgcn_wave_barrier();

  acc[0] = acc[1] = 0.f;
  auto block = [&](int k0, auto tail) __attribute__((always_inline)) {
#pragma unroll
    for (int u4 = 0; u4 < kQueue; u4 += 4) {
      const f32x4 w4 = *(const f32x4*)&kw[k0 + u4];
#pragma unroll
      for (int u = u4; u < u4 + 4; ++u) {
        // in the last block a row past the last split is zeroed: acc + 0 * 0 = acc exactly
        // (acc is never -0)
        const uint32_t v = (decltype(tail)::value && k0 + u >= n) ? 0u : qv[u];
        float x0, x1;
        if constexpr (LDT == MLA_DTYPE_BF16) {
          x0 = __builtin_bit_cast(float, v << 16);
          x1 = __builtin_bit_cast(float, v & 0xffff0000u);
        } else {
          const f16x2 h = __builtin_bit_cast(f16x2, v);
          x0 = (float)h[0];
          x1 = (float)h[1];
        }
        acc[0] += w4[u - u4] * x0;
        acc[1] += w4[u - u4] * x1;
        qv[u] = load_next();
      }
    }
  };
  for (int k0 = 0; k0 < n; k0 += kQueue) {
    if (k0 + kQueue <= n)  // uniform
      block(k0, std::false_type{});
    else
      block(k0, std::true_type{});
  }
  return lse2;
}

// One wave per (sequence, row).  DEEP (chosen by the host when the batch is small next to the
// part count, so sequences have many splits and the grid is small): one wave per workgroup and
// grid.z = 4, the quarter of the row the wave merges when the row has kFewSplits < n <=
// kDeepSplits splits (merge_many_splits); other rows are merged whole by quarter 0.  Otherwise
// four waves per workgroup, for large batches of rows with few splits each.
template <int DT, typename PT, bool SCALED, bool DEEP = false>
__global__ __launch_bounds__(DEEP ? 64 : 256) void mla_combine_kernel(const PT* __restrict__ ws_o,
                                                          const float* __restrict__ ws_scale,
                                                          const float* __restrict__ ws_lse,
                                                          const int32_t* __restrict__ splits,
                                                          int rows, int heads, int s_q,
                                                          uint16_t* __restrict__ out,
                                                          int64_t o_sb, int64_t o_ss, int64_t o_sh,
                                                          float* __restrict__ lse_out,
                                                          int copy_single) {
  constexpr int W = DEEP ? 1 : 4;  // waves (rows) per workgroup
  __shared__ __attribute__((aligned(16))) char smem[DEEP ? kDeepLds : W * 64 * 4];
  float* w_sh = (float*)smem + 64 * (threadIdx.x >> 6);  // the wave's 64 weights (merge_splits_wave)
  const int b = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.y * W + wave;
  if (row >= rows) return;
  const int base = splits[b];
  const int n = splits[b + 1] - base;
  if (n < 1 || (n == 1 && !copy_single)) return;
  const int s = row / heads;
  const int h = row - s * heads;
  uint16_t* dst = out + b * o_sb + s * o_ss + h * o_sh;
  float* lse_dst = lse_out != nullptr ? lse_out + ((int64_t)b * heads + h) * s_q + s : nullptr;
  if constexpr (DEEP && std::is_same<PT, uint16_t>::value) {
    const int q = blockIdx.z;
    if (n > kFewSplits && n <= kDeepSplits) {  // uniform
      float acc2[2];
      const float lse2 = merge_many_splits<DT, SCALED>(ws_o, ws_scale, ws_lse, base, n, rows, row, q, lane, smem, acc2);
      *(uint32_t*)(dst + 128 * q + 2 * lane) = pack2<DT>(acc2[0], acc2[1]);
      if (q == 0 && lane == 0 && lse_dst != nullptr) *lse_dst = lse2 * kLn2;
      return;
    }
    if (q != 0) return;
  }
  float acc[8];
  float lse2;
  if constexpr (std::is_same<PT, uint16_t>::value) {
    if (n <= kFewSplits)  // uniform
      lse2 = merge_few_splits<DT, SCALED>(ws_o, ws_scale, ws_lse, base, n, rows, row, lane, acc);
    else
      lse2 = merge_splits_wave<DT, PT, SCALED>(ws_o, ws_scale, ws_lse, base, n, rows, row, lane, w_sh, acc);
  } else {
    lse2 = merge_splits_wave<DT, PT, SCALED>(ws_o, ws_scale, ws_lse, base, n, rows, row, lane, w_sh, acc);
  }
  *(i32x4*)(dst + lane * 8) = i32x4{(int)pack2<DT>(acc[0], acc[1]), (int)pack2<DT>(acc[2], acc[3]),
                                    (int)pack2<DT>(acc[4], acc[5]), (int)pack2<DT>(acc[6], acc[7])};
  if (lane == 0 && lse_dst != nullptr) *lse_dst = lse2 * kLn2;
}

// ---------------------------------------------------------------------------------------
// absorbed value projection with the combine fused into its prologue
// ---------------------------------------------------------------------------------------
// v[m, h, :] = o[m, h, :] . W_UV[h]  (m = b * s_q + s, o the merged latent output, W_UV[h] the
// head's 512 x kVDim up-projection, given k-blocked: w_blk[h][kb][n][kk] = W_UV[h][32kb + kk][n],
// so the B operand of one MFMA k-step for 16 columns is one contiguous KiB).  One workgroup of
// 4 waves per (head, tile of 16 rows); wave w merges rows 4w .. 4w+3 and owns output columns
// 32w .. 32w+31.  The kernel is a chain of dependent memory round trips, so it is arranged to
// have few:
//  1. the rows' split ranges are loaded;
//  2. the lse of each row's first 64 splits and the partial rows of its first kPF splits are
//     loaded together (the partials do not depend on the weights); the rows are merged into LDS
//     as bf16, never written to HBM (a single-split row is read from `out`, where the decode
//     wrote it).  Each row follows the combine's arithmetic operation for operation
//     (merge_splits_wave): the same lse (lane-strided max and sum, xor-butterfly), the same
//     weights, the same fma chain in split order;
//  3. the wave's W_UV slab (32 columns, 128 registers) is loaded in one round trip and 2 MFMA
//     tiles form the 16 x kVDim product.
// At most 256 registers (178 used): two workgroups per CU.  At three (168 registers) the
// compiler spilled 28 of them to scratch and the kernel ran 4-21% slower.  (Measured
// alternatives: loading W_UV before the merge, and 32-row workgroups of 8 waves that preload
// their 16-column slabs, were no faster; the [h][n][k] layout, 16 half-lines per load, cost
// 3 us more at 128 heads x 64 rows.)
constexpr int kVDim = 128;
constexpr int kAbsRows = 16;
struct AbsorbParams {
  const uint16_t* ws_o;   // [slots, rows, 512] fp16 partials, chunk c times 2^e
  const float* ws_scale;  // [slots, rows, 4] the chunks' 2^-e
  const float* ws_lse;    // [slots, rows] log2
  const int32_t* splits;
  const uint16_t* out;   // single-split rows
  int64_t o_sb, o_ss, o_sh;
  const uint16_t* w_blk;  // [H, 16, kVDim, 32]
  uint16_t* v;           // [M, H, kVDim]
  float* lse;            // [B, H, s_q] natural log, or null
  int32_t m_rows, s_q, heads, rows;
  int32_t premerged;     // 1: the combine kernel already wrote every row to `out` (and its lse)
};

template <int DT>
__global__ __launch_bounds__(256, 2) void mla_combine_absorb_kernel(AbsorbParams a) {
  constexpr int RT = kAbsRows;     // rows per workgroup
  constexpr int kPitch = kDV + 8;  // 16-bit elements; 1040-byte rows keep the A reads conflict-free
  constexpr int R = RT / 4;        // rows merged by one wave
  constexpr int NT = 2;            // 16-column MFMA tiles per wave
  constexpr int KS = kDV / 32;     // MFMA k-steps
  constexpr int kPF = 2;           // partial rows per row loaded in one round trip
  // a group of kPF splits must not cross a 64-split weight window (w_sh holds one window);
  // 4 spills 61 registers at this launch bound
  static_assert(64 % kPF == 0, "kPF divides the weight window");
  __shared__ __attribute__((aligned(16))) uint16_t a_sh[RT * kPitch];
  __shared__ float w_sh[RT][64];
  const int h = blockIdx.x;
  const int m0 = blockIdx.y * RT;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, li = lane & 15;

  // ---- 1. split ranges of the wave's rows
  const int r0 = wave * R;
  const int64_t split_stride = (int64_t)a.rows * kDV;
  int n[R];
  const uint16_t* src1[R];  // single-split rows: the decode's output (input dtype)
  const uint16_t* src[R];   // split rows: scaled fp16 partials
  const float* scp[R];      // their scales (this lane's chunk, lane / 16)
  const float* lsep[R];
  int nmax = 0;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int m = m0 + r0 + i;
    n[i] = 0;
    src1[i] = a.out;
    src[i] = a.ws_o;
    scp[i] = a.ws_scale;
    lsep[i] = a.ws_lse;
    if (m < a.m_rows) {
      const int b = m / a.s_q, s = m - b * a.s_q;
      const int row = s * a.heads + h;
      const int base = a.splits[b];
      n[i] = a.splits[b + 1] - base;
      if (a.premerged && n[i] > 1) n[i] = 1;  // the merged row is in `out`, its lse written
      if (n[i] == 1) {
        src1[i] = a.out + b * a.o_sb + s * a.o_ss + h * a.o_sh + lane * 8;
      } else {
        src[i] = a.ws_o + ((int64_t)base * a.rows + row) * kDV + lane * 8;
        scp[i] = a.ws_scale + ((int64_t)base * a.rows + row) * 4 + (lane >> 4);
        lsep[i] = a.ws_lse + (int64_t)base * a.rows + row;
      }
    }
    nmax = n[i] > nmax ? n[i] : nmax;
  }
  // the eight values of split u of row i owned by this lane, widened to fp32, and their scale
  // (1 for a single-split row; branches are wave-uniform: all lanes work on the same row)
  auto load_row = [&](int u, int i, float (&xv)[8], float& us) __attribute__((always_inline)) {
    if (n[i] == 1) {
      cvt8<DT>(*(const i32x4*)src1[i], xv);
      us = 1.f;
    } else {
      load8<MLA_DTYPE_F16>(src[i] + u * split_stride, xv);
      us = scp[i][(int64_t)u * a.rows * 4];
    }
  };

  // ---- 2. partial rows of the first kPF splits, and the lse of split `lane`, in one round trip
  float x[kPF][R][8], us[kPF][R];
#pragma unroll
  for (int u = 0; u < kPF; ++u)
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (u < n[i]) load_row(u, i, x[u][i], us[u][i]);
  float l0[R], lse2[R];
#pragma unroll
  for (int i = 0; i < R; ++i) l0[i] = (n[i] > 1 && lane < n[i]) ? lsep[i][(int64_t)lane * a.rows] : 0.f;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    lse2[i] = -INFINITY;
    if (n[i] > 1) {
      float mx = -INFINITY;
      if (lane < n[i]) mx = fmaxf(mx, l0[i]);
      for (int k = lane + 64; k < n[i]; k += 64) mx = fmaxf(mx, lsep[i][(int64_t)k * a.rows]);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      float sum = 0.f;
      if (mx != -INFINITY) {
        if (lane < n[i]) sum += fast_exp2(l0[i] - mx);
        for (int k = lane + 64; k < n[i]; k += 64) sum += fast_exp2(lsep[i][(int64_t)k * a.rows] - mx);
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
      lse2[i] = sum > 0.f ? mx + __log2f(sum) : -INFINITY;
      if (lane == 0 && a.lse != nullptr) {
        const int m = m0 + r0 + i;
        const int b = m / a.s_q, s = m - b * a.s_q;
        a.lse[((int64_t)b * a.heads + h) * a.s_q + s] = lse2[i] * kLn2;
      }
    }
  }
  float acc[R][8];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;
  for (int k0 = 0; k0 < nmax; k0 += 64) {
    const int k = k0 + lane;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      float w = 0.f;
      if (n[i] == 1) {
        w = 1.f;  // fma(1, x, 0) = x: the single-split row as the decode wrote it
      } else if (k < n[i] && lse2[i] != -INFINITY) {
        w = fast_exp2((k0 == 0 ? l0[i] : lsep[i][(int64_t)k * a.rows]) - lse2[i]);
      }
      w_sh[r0 + i][lane] = w;
    }
    __builtin_amdgcn_wave_barrier();
    const int kn = nmax - k0 < 64 ? nmax - k0 : 64;
    for (int kb = 0; kb < kn; kb += kPF) {
      if (k0 + kb > 0) {
#pragma unroll
        for (int u = 0; u < kPF; ++u)
#pragma unroll
          for (int i = 0; i < R; ++i)
            if (k0 + kb + u < n[i]) load_row(k0 + kb + u, i, x[u][i], us[u][i]);
      }
#pragma unroll
      for (int u = 0; u < kPF; ++u)
#pragma unroll
        for (int i = 0; i < R; ++i)
          if (k0 + kb + u < n[i]) {
            const float wk = w_sh[r0 + i][kb + u] * us[u][i];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] += wk * x[u][i][j];
          }
    }
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
    *(i32x4*)&a_sh[(r0 + i) * kPitch + lane * 8] =
        i32x4{(int)pack2<DT>(acc[i][0], acc[i][1]), (int)pack2<DT>(acc[i][2], acc[i][3]),
              (int)pack2<DT>(acc[i][4], acc[i][5]), (int)pack2<DT>(acc[i][6], acc[i][7])};

  // ---- 3. this wave's B fragments (8 consecutive k of one column n) in one round trip, then
  //         the 16 x kVDim product
  const uint16_t* wb0 = a.w_blk + (int64_t)h * kVDim * kDV + (32 * wave + li) * 32 + 8 * g;
  i32x4 bf[KS][NT];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) bf[ks][nt] = *(const i32x4*)(wb0 + (ks * kVDim + 16 * nt) * 32);
  __syncthreads();
  f32x4 c[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) c[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const i32x4 af = *(const i32x4*)&a_sh[li * kPitch + 32 * ks + 8 * g];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) c[nt] = mfma32<DT>(af, bf[ks][nt], c[nt]);
  }
  // lane (g, li) holds rows 4g .. 4g+3 of column li of each tile
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 4 * g + r;
      if (m < a.m_rows) {
        const float v = c[nt][r];
        const uint32_t pk = pack2<DT>(v, v);
        a.v[((int64_t)m * a.heads + h) * kVDim + 32 * wave + 16 * nt + li] = (uint16_t)(pk & 0xFFFF);
      }
    }
}

// ---------------------------------------------------------------------------------------
// tile schedule on the device: one workgroup of four waves.
//   1. page counts (coalesced) and their block-wide prefix sums of pages + f (32-bit while
//      the total is below 2^30);
//   2. one wave per candidate payload walks the sequences in windows of 64 (mla_sched.h's
//      closed form gives the packing state between resets): every lane looks up to 8
//      sequences ahead for the reset that would follow it, the wave follows these links from
//      reset to reset with scalar reads, and a ballot over the window finds the next reset
//      where a link is missing.  It records the state at every window start and the window's
//      reset lanes;
//   3. each wave takes whole windows: every lane rebuilds the state entering its sequence from
//      the window's record (last reset below it, a wave prefix sum of the part increments)
//      and writes the records of the parts that begin inside it.
// With no pages at all or a total of 2^30 pages or more, a serial pass per candidate replaces
// steps 2 and 3.  Either way the schedule is exactly the host's.  Forced splits: slot counts,
// their prefix sums, one thread per record.
// ---------------------------------------------------------------------------------------
constexpr int kMetaMaxBatch = 16384;
constexpr int kMetaThreads = 256;
constexpr int kMetaWaves = kMetaThreads / 64;
constexpr int kMetaMaxCand = 8;
constexpr int kMetaMaxWin = kMetaMaxBatch / kWalkWin;
static_assert(kWalkWin == 64, "a walk window is one wave");

// Exclusive prefix over the workgroup of one int64 per thread (and the total).
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t v, int64_t* wsum_sh, int64_t* total) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  int64_t inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t o = __shfl_up(inc, off);
    if (lane >= off) inc += o;
  }
  if (lane == 63) wsum_sh[wave] = inc;
  __syncthreads();
  int64_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kMetaWaves; ++w) {
    const int64_t x = wsum_sh[w];
    before += w < wave ? x : 0;
    all += x;
  }
  __syncthreads();  // wsum_sh is free again
  *total = all;
  return before + inc - v;
}

// Inclusive prefix of one int over the wave.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(v, off);
    if (lane >= off) v += o;
  }
  return v;
}

// Orders this wave's LDS accesses across lanes: a wave-scope fence (waits for the wave's LDS
// operations) and a code-motion barrier, so a lane may read what other lanes just wrote.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The walk of one candidate payload T by one wave (S: prefix sums in LDS, batch + 1 entries;
// sig: the wave's scratch for kWalkWin + kWalkLook residues).  Writes the window entries and
// reset masks; returns the final part index, -1 if T cannot place a sequence (c < 1).  The
// same steps as walk_payload_host in mla_sched.h; the lookahead runs on every lane at once,
// without branches.
__device__ int walk_payload_wave(const int32_t* S, int batch, int T, int f, WalkEntry* ent, uint64_t* msk,
                                 int* sig) {
  const int lane = threadIdx.x & 63;
  const int c = T - f;
  if (c < 1) return -1;
  const uint32_t cu = (uint32_t)c;
  const int f1 = (int)((uint32_t)(f + 1) % cu);
  int rs = 0, rsig = 0, p = 0, w = 0;  // last reset: prefix, residue, the part it opened; resets
  int pend = -1, pend_inc = 0;         // a reset in the next window, reached by a link
  const int nwin = (batch + kWalkWin - 1) / kWalkWin;
#pragma unroll 1
  for (int win = 0; win < nwin; ++win) {
    const int base = win * kWalkWin;
    if (lane == 0) ent[win] = WalkEntry{rs, p, w};
    const int i = base + lane;
    const bool in = i < batch;
    const int Si = S[in ? i : batch];
    const int Sn = S[in ? i + 1 : batch];
    const int si = (int)((uint32_t)Si % cu);
    wave_lds_sync();  // the previous window's reads of sig are done
    sig[lane] = si;
    if (lane < kWalkLook) {
      const int k = base + kWalkWin + lane;
      sig[kWalkWin + lane] = (int)((uint32_t)S[k < batch ? k : batch] % cu);
    }
    wave_lds_sync();  // other lanes' residues are visible
    // lookahead of every lane: all operands loaded first, then a branch-free test per step
    int Sv[kWalkLook + 1], sv[kWalkLook];
#pragma unroll
    for (int d = 0; d <= kWalkLook; ++d) Sv[d] = S[min(i + 1 + d, batch)];  // S[i+1 .. i+9]
#pragma unroll
    for (int d = 0; d < kWalkLook; ++d) sv[d] = sig[lane + 1 + d];
    int d_l = 0, a_l = 0;
#pragma unroll
    for (int d = 1; d <= kWalkLook; ++d) {
      const int Sk = Sv[d - 1], Skn = Sv[d];
      const int A = Sk - Si;
      const int e2 = mod_sub(mod_sub(sv[d - 1], si, c), f1, c);
      const int rem = A <= T ? T - A : c - 1 - e2;
      const bool hit = (d_l == 0) & (i + d < batch) & (rem <= f) & (rem < Skn - Sk);
      d_l = hit ? d : d_l;
      a_l = hit ? A : a_l;
    }
    const int inc_l = d_l > 0 ? walk_parts(a_l, T, f, c) + 1 : 0;
    uint64_t mask = 0;
    int cur = -1;  // lane of the last reset in this window (wave-uniform)
    if (pend >= 0) {
      cur = pend;
      p += pend_inc;
      w += 1;
      mask |= 1ull << cur;
      pend = -1;
    }
#pragma unroll 1
    for (;;) {
      int from = 0;
      if (cur >= 0) {
        int d = __builtin_amdgcn_readlane(d_l, cur);
#pragma unroll 1
        while (d > 0 && cur + d < kWalkWin) {
          p += __builtin_amdgcn_readlane(inc_l, cur);
          w += 1;
          cur += d;
          mask |= 1ull << cur;
          d = __builtin_amdgcn_readlane(d_l, cur);
        }
        rs = __builtin_amdgcn_readlane(Si, cur);
        rsig = __builtin_amdgcn_readlane(si, cur);
        if (d > 0) {
          pend = cur + d - kWalkWin;
          pend_inc = __builtin_amdgcn_readlane(inc_l, cur);
          break;
        }
        from = cur + kWalkLook + 1;
      }
      if (from >= kWalkWin) break;
      const int A = Si - rs;
      const int e2 = mod_sub(mod_sub(si, rsig, c), f1, c);
      const int rem = A <= T ? T - A : c - 1 - e2;
      const bool r = in & (i > 0) & (lane >= from) & (rem <= f) & (rem < Sn - Si);
      const uint64_t m = __ballot(r);
      if (m == 0) break;
      cur = __builtin_ctzll(m);
      const int Sj = __builtin_amdgcn_readlane(Si, cur);
      p += walk_parts(Sj - rs, T, f, c) + 1;
      w += 1;
      rs = Sj;
      rsig = __builtin_amdgcn_readlane(si, cur);
      mask |= 1ull << cur;
    }
    if (lane == 0) msk[win] = mask;
  }
  return p + walk_parts(S[batch] - rs, T, f, c);
}

__global__ __launch_bounds__(kMetaThreads) void mla_metadata_kernel(
    const int32_t* __restrict__ seqlens, int batch, int num_parts, int f, int min_payload,
    int forced, int32_t* __restrict__ sched, int32_t* __restrict__ splits) {
  // page counts; on the walk path overwritten in place by the exclusive prefix of pages + f
  __shared__ int32_t s_sh[kMetaMaxBatch + 1];
  // walk: entries and reset masks per candidate and window; serial pass: the packing state per
  // candidate at every chunk start (never live together)
  constexpr int kWalkBytes = kMetaMaxCand * kMetaMaxWin * (int)(sizeof(WalkEntry) + sizeof(uint64_t));
  constexpr int kSerialBytes = kMetaMaxCand * kMetaThreads * (int)sizeof(PackState);
  __shared__ __attribute__((aligned(16))) uint8_t u_sh[kWalkBytes > kSerialBytes ? kWalkBytes : kSerialBytes];
  uint64_t (*msk_sh)[kMetaMaxWin] = reinterpret_cast<uint64_t (*)[kMetaMaxWin]>(u_sh);
  WalkEntry (*ent_sh)[kMetaMaxWin] =
      reinterpret_cast<WalkEntry (*)[kMetaMaxWin]>(u_sh + kMetaMaxCand * kMetaMaxWin * sizeof(uint64_t));
  PackState (*st_sh)[kMetaThreads] = reinterpret_cast<PackState (*)[kMetaThreads]>(u_sh);
  __shared__ PackState fin_sh[kMetaMaxCand];
  __shared__ int64_t red_sh[kMetaWaves];
  __shared__ int flag_sh[kMetaWaves];
  __shared__ int sig_sh[kMetaWaves][kWalkWin + kWalkLook];  // each wave's residues (walk)
  __shared__ int ok_sh[kMetaMaxCand];
  __shared__ int last_sh[kMetaMaxCand];
  __shared__ int last_part_sh;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;

  for (int i = t; i < batch; i += kMetaThreads) s_sh[i] = pages_of(seqlens[i]);
  __syncthreads();
  // each thread's contiguous chunk of sequences (for the prefix sums)
  const int chunk = (batch + kMetaThreads - 1) / kMetaThreads;
  const int b0 = min(batch, t * chunk), b1 = min(batch, b0 + chunk);

  if (forced > 0) {
    int64_t cnt = 0;
    for (int b = b0; b < b1; ++b) cnt += forced_count(s_sh[b], forced);
    int64_t slots;
    int64_t cum = block_exclusive_scan(cnt, red_sh, &slots);
    if (t == 0) splits[0] = 0;
    for (int b = b0; b < b1; ++b) {
      cum += forced_count(s_sh[b], forced);
      splits[b + 1] = (int32_t)cum;
    }
    const int nrec = batch * forced;  // == num_parts (host-checked)
    for (int r = t; r < nrec; r += kMetaThreads) {
      const int b = r / forced;
      forced_record(b, r - b * forced, s_sh[b], forced, sched);
    }
    return;
  }

  // chunk sums fit 31 bits (<= 64 sequences of < 2^25 pages); a chunk of 2^22 or more may
  // take the total past 2^30, which routes to the serial pass (64-bit where needed)
  int cost = 0, any = 0;
  for (int b = b0; b < b1; ++b) {
    cost += s_sh[b] + f;
    any |= s_sh[b];
  }
  const int flags = (any != 0 ? 1 : 0) | (cost >= (1 << 22) ? 2 : 0);
  int incl = wave_inclusive_scan(cost);
  const int wflags = (__ballot(flags & 1) != 0 ? 1 : 0) | (__ballot(flags & 2) != 0 ? 2 : 0);
  if (lane == 63) {
    red_sh[wave] = incl;
    flag_sh[wave] = wflags;
  }
  __syncthreads();
  int before = incl - cost, total32 = 0, all_flags = 0;
#pragma unroll
  for (int w = 0; w < kMetaWaves; ++w) {
    before += w < wave ? (int)red_sh[w] : 0;
    total32 += (int)red_sh[w];
    all_flags |= flag_sh[w];
  }
  const bool walk = all_flags == 1;  // pages somewhere, total below 2^30
  int64_t total = total32;
  if (!walk) {
    __syncthreads();  // red_sh is reused
    int64_t b64;
    block_exclusive_scan(cost, red_sh, &b64);
    total = b64;
  }
  int64_t lo, hi;
  payload_bounds(total, num_parts, f, &lo, &hi);
  const int ncand = min_payload ? (int)(hi - lo) + 1 : 1;  // <= kMetaMaxCand (host-checked)
  int best = ncand - 1;  // the largest candidate (hi) always fits
  int64_t T;
  const auto emit = [&](int p, int b, int page, int split) {
    if (p < num_parts) {
      int32_t* rec = sched + p * kSchedWords;
      rec[0] = b;
      rec[1] = page;
      rec[4] = split;
    }
    if (p - 1 < num_parts) {
      sched[(p - 1) * kSchedWords + 2] = b;
      sched[(p - 1) * kSchedWords + 3] = page;
    }
  };
  if (t == 0) {  // part 0 begins at the first page; its end is written by whoever closes it
    sched[0] = 0;
    sched[1] = 0;
    sched[4] = 0;
    splits[0] = 0;
  }

  if (walk) {
    // ---- prefix sums in place (each thread owns its chunk)
    int run = before;
    for (int b = b0; b < b1; ++b) {
      const int n = s_sh[b];
      s_sh[b] = run;
      run += n + f;
    }
    if (t == 0) s_sh[batch] = total32;
    __syncthreads();
    for (int ci = wave; ci < ncand; ci += kMetaWaves) {  // uniform per wave
      const int fin = walk_payload_wave(s_sh, batch, (int)(min_payload ? lo + ci : hi), f, ent_sh[ci], msk_sh[ci],
                                        sig_sh[wave]);
      if (lane == 0) {
        ok_sh[ci] = fin >= 0 && fin < num_parts;
        last_sh[ci] = fin;
      }
    }
    __syncthreads();
    for (int i = ncand - 1; i >= 0; --i)
      if (ok_sh[i]) best = i;
    T = min_payload ? lo + best : hi;
    const int Tb = (int)T, c = Tb - f;
    const int nwin = (batch + kWalkWin - 1) / kWalkWin;
    for (int win = wave; win < nwin; win += kMetaWaves) {  // uniform per wave
      const int m = win * kWalkWin + lane;
      const bool in = m < batch;
      const WalkEntry e = ent_sh[best][win];
      const uint64_t mask = msk_sh[best][win];
      const uint64_t below = mask & ((1ull << lane) - 1);
      const int Sm = in ? s_sh[m] : 0;
      const int Sprev = below != 0 ? s_sh[win * kWalkWin + 63 - __builtin_clzll(below)] : e.rs;
      const int inc = ((mask >> lane) & 1) ? walk_parts(Sm - Sprev, Tb, f, c) + 1 : 0;
      const int pinc = wave_inclusive_scan(inc);  // part increments of the resets up to this lane
      if (in) {
        const int A = Sm - Sprev;
        int part = e.p + pinc - inc + walk_parts(A, Tb, f, c);
        int remain = walk_remain(A, Tb, f, c);
        int cum = part + m - (e.w + __builtin_popcountll(below));
        pack_sequence_emit32(m, s_sh[m + 1] - Sm - f, Tb, f, remain, part, cum, emit);
        splits[m + 1] = cum;
      }
    }
    if (t == 0) last_part_sh = last_sh[best];
  } else {
    // ---- serial pass per candidate (s_sh holds page counts)
    const int nchunks = (batch + chunk - 1) / chunk;  // chunks that hold sequences, <= kMetaThreads
    if (t < ncand) {
      // one sequence after another, the next one's page count read from LDS while this one is
      // packed; 32-bit steps while every quantity fits 31 bits, else 64-bit
      const int64_t Tc = min_payload ? lo + t : hi;
      PackState st{Tc, 0, 0};
      bool ok = true;
      int n_next = s_sh[0];
      if (total < (1ll << 30)) {
        int remain = (int)Tc, part = 0, cum = 0;
        for (int c = 0; c < nchunks; ++c) {
          st_sh[t][c] = PackState{remain, part, cum};
          const int e = min(batch, (c + 1) * chunk);
          for (int b = c * chunk; b < e; ++b) {
            const int n = n_next;
            n_next = s_sh[b + 1 < batch ? b + 1 : b];
            if (ok) ok = pack_sequence32(n, (int)Tc, f, remain, part, cum) && part < num_parts;
          }
        }
        st = PackState{remain, part, cum};
      } else {
        for (int c = 0; c < nchunks; ++c) {
          st_sh[t][c] = st;
          const int e = min(batch, (c + 1) * chunk);
          for (int b = c * chunk; b < e; ++b) {
            const int n = n_next;
            n_next = s_sh[b + 1 < batch ? b + 1 : b];
            if (ok) ok = pack_sequence(b, n, Tc, f, st, NoEmit{}) && st.part < num_parts;
          }
        }
      }
      fin_sh[t] = st;  // the state every empty chunk starts (and ends) in
      ok_sh[t] = ok ? 1 : 0;
    }
    __syncthreads();
    for (int i = ncand - 1; i >= 0; --i)
      if (ok_sh[i]) best = i;
    T = min_payload ? lo + best : hi;
    PackState st = t < nchunks ? st_sh[best][t] : fin_sh[best];
    for (int b = b0; b < b1; ++b) {
      pack_sequence(b, s_sh[b], T, f, st, emit);
      splits[b + 1] = st.cum;
    }
    if (t == kMetaThreads - 1) last_part_sh = st.part;  // the last chunk ends at the final state
  }
  __syncthreads();
  const int last = last_part_sh;
  for (int p = t; p < num_parts; p += kMetaThreads) {
    int32_t* rec = sched + p * kSchedWords;
    if (p > last) {
      sched_write(rec, batch, 0, batch, 0, 0);
    } else {
      if (p == last) {
        rec[2] = batch;
        rec[3] = 0;
      }
      rec[5] = 0;
      rec[6] = 0;
      rec[7] = 0;
    }
  }
}

// mla_launch's schedule: the reference's frozen shape (one sequence of kHandCtx tokens) cut
// into ns forced splits, written by one thread into the caller's scratch.
constexpr int kHandCtx = 8192;
constexpr int kHandHeads = 16;
__global__ __launch_bounds__(64) void mla_launch_sched_kernel(int32_t* seqlens, int32_t* sched,
                                                              int32_t* splits, int ns) {
  if (threadIdx.x == 0) {
    seqlens[0] = kHandCtx;
    schedule_forced(seqlens, 1, ns, sched, splits);
  }
}

}  // namespace mla

// =========================================================================================
// C ABI
// =========================================================================================
namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

struct Variant {
  int nw, ht, nstage;
  bool ws;  // wave split: the waves share one row tile and take turns over the stages
  int rows() const { return ws ? 16 * ht : nw * 16 * ht; }
  int lds() const { return (ws ? nw : nstage) * mla::kStageBytes; }
};

// A wave owns one 16-row tile (72 VGPRs of query, 128 AGPRs of fp32 output) or two (32 rows:
// 144 VGPRs of query, 256 AGPRs of output, and every K / V fragment read from LDS feeds two
// MFMAs).
//  - up to 16 rows: four waves take turns over the stages of one tile, each with its own
//    36 KiB slot (one workgroup per CU).  Each wave waits for its own stage while the others
//    compute, which keeps 4 x 36 KiB of loads in flight per CU (one wave alone could hold at
//    most 63 KiB: vmcnt), and the merge at the end of a segment leaves one partial per
//    workgroup instead of one per wave: a quarter of the split partials (their stores cost
//    far more than their bytes suggest when they interleave with the KV reads) and a quarter
//    of the page-granular imbalance between parts;
//  - up to 32 rows: one wave of two tiles per workgroup with its own 36 KiB stage buffer,
//    four workgroups per CU (the wave-split form of two tiles spills registers);
//  - up to 64 rows: four waves of one tile each sharing a 4-stage ring;
//  - above 64 rows: four waves of two tiles (128 rows) sharing a 3-stage ring, so each KV
//    stage is read into LDS once for all 128 rows; more rows use ceil(rows/128) head blocks.
Variant pick_variant(int rows) {
  if (rows <= 16) return {4, 1, 1, true};
  if (rows <= 32) return {1, 2, 1, false};
  if (rows <= 64) return {4, 1, 4, false};
  return {4, 2, 3, false};
}

int wgs_per_cu(const Variant& v) {
  const int lds = v.lds();
  int by_lds = (160 * 1024) / lds;
  if (by_lds < 1) by_lds = 1;
  const int per_simd = mla::waves_per_simd(v.nw, v.ht, v.nstage, v.ws);
  const int by_waves = 4 * per_simd / v.nw > 0 ? 4 * per_simd / v.nw : 1;
  return by_lds < by_waves ? by_lds : by_waves;
}

int cu_count_current() {
  static std::once_flag once;
  static int cached = 256;
  std::call_once(once, [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cached = n;
  });
  return cached;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int64_t ws_lse_bytes(int64_t slots, int64_t rows) {
  return ((slots * rows * 4) + 255) / 256 * 256;
}
int64_t ws_scale_bytes(int64_t slots, int64_t rows) {
  return ((slots * rows * 4 * 4) + 255) / 256 * 256;
}

template <int DT, int NW, int HT, int NS, bool WS, bool KV8 = false, bool SPARSE = false>
hipError_t launch_main(const mla::KParams& kp, int head_blocks, hipStream_t st) {
  hipLaunchKernelGGL((mla::mla_splitkv_kernel<DT, NW, HT, NS, WS, KV8, SPARSE>), dim3(kp.num_parts, head_blocks),
                     dim3(NW * 64), 0, st, kp.sched, kp);
  return hipGetLastError();
}

// The 64- and 128-row dense decodes run the wide kernel (PV split by dims across the waves)
// unless MLA_WIDE=0 selects the one-ring four-wave kernel (kept for the fp8 and sparse paths).
bool wide_enabled() {
  static std::once_flag once;
  static bool on = true;
  std::call_once(once, [] {
    const char* e = getenv("MLA_WIDE");
    on = !(e != nullptr && e[0] == '0');
  });
  return on;
}

template <int DT, int HT, bool FUSED>
void launch_wide_form(const mla::KParams& kp, int head_blocks, hipStream_t st) {
  const int wgs = kp.num_parts * head_blocks;
  if (wgs % 8 == 0) {  // XCD-blocked 1-D grid (see the kernel)
    hipLaunchKernelGGL((mla::mla_wide_kernel<DT, HT, FUSED>), dim3(wgs), dim3(256), 0, st, kp.sched, head_blocks, wgs / 8,
                       kp);
  } else {
    hipLaunchKernelGGL((mla::mla_wide_kernel<DT, HT, FUSED>), dim3(kp.num_parts, head_blocks), dim3(256), 0, st, kp.sched,
                       0, 0, kp);
  }
}

// The fused-rope form for the 128-row kernel only (the 64-row one measured 2% slower with it).
template <int DT, int HT>
hipError_t launch_wide(const mla::KParams& kp, int head_blocks, hipStream_t st) {
  if constexpr (HT == 2) {
    if (kp.rope_fused) {
      launch_wide_form<DT, HT, true>(kp, head_blocks, st);
      return hipGetLastError();
    }
  }
  launch_wide_form<DT, HT, false>(kp, head_blocks, st);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_main_dt(const Variant& v, const mla::KParams& kp, int head_blocks, hipStream_t st) {
  if (kp.indices != nullptr) {  // sparse (top-k) decode
    if constexpr (DT == MLA_DTYPE_BF16) {
      if (kp.kv_scale != nullptr) {  // over the fp8 latent cache
        if (v.ws) return launch_main<DT, 4, 1, 1, true, true, true>(kp, head_blocks, st);
        if (v.nw == 1) return launch_main<DT, 1, 2, 1, false, true, true>(kp, head_blocks, st);
        if (v.ht == 1) return launch_main<DT, 4, 1, 4, false, true, true>(kp, head_blocks, st);
        return launch_main<DT, 4, 2, 3, false, true, true>(kp, head_blocks, st);
      }
    }
    if (v.ws) return launch_main<DT, 4, 1, 1, true, false, true>(kp, head_blocks, st);
    if (v.nw == 1) return launch_main<DT, 1, 2, 1, false, false, true>(kp, head_blocks, st);
    if (v.ht == 1) return launch_main<DT, 4, 1, 4, false, false, true>(kp, head_blocks, st);
    return launch_main<DT, 4, 2, 3, false, false, true>(kp, head_blocks, st);
  }
  if constexpr (DT == MLA_DTYPE_BF16) {
    if (kp.kv_scale != nullptr) {  // fp8 latent cache
      if (v.ws) return launch_main<DT, 4, 1, 1, true, true>(kp, head_blocks, st);
      if (v.nw == 1) return launch_main<DT, 1, 2, 1, false, true>(kp, head_blocks, st);
      if (v.ht == 1) return launch_main<DT, 4, 1, 4, false, true>(kp, head_blocks, st);
      return launch_main<DT, 4, 2, 3, false, true>(kp, head_blocks, st);
    }
  }
  if (v.ws) return mla::launch_ws_dense<DT>(kp, head_blocks, st);  // mla_decode_ws.hip
  if (v.nw == 1) return launch_main<DT, 1, 2, 1, false>(kp, head_blocks, st);
  if (wide_enabled()) return v.ht == 1 ? launch_wide<DT, 1>(kp, head_blocks, st) : launch_wide<DT, 2>(kp, head_blocks, st);
  if (v.ht == 1) return launch_main<DT, 4, 1, 4, false>(kp, head_blocks, st);
  return launch_main<DT, 4, 2, 3, false>(kp, head_blocks, st);
}

int validate(const mla_decode_args* a, int64_t* need_ws) {
  if (a == nullptr) return fail(MLA_ERR_INVALID, "args is NULL");
  if (a->batch < 1 || a->s_q < 1 || a->heads_q < 1)
    return fail(MLA_ERR_INVALID, "batch, s_q and heads_q must be >= 1");
  if (a->heads_k != 1) return fail(MLA_ERR_UNSUPPORTED, "only heads_k == 1 (one latent KV head) is supported");
  if (a->dtype != MLA_DTYPE_BF16 && a->dtype != MLA_DTYPE_F16)
    return fail(MLA_ERR_INVALID, "dtype must be MLA_DTYPE_BF16 or MLA_DTYPE_F16");
  if ((int64_t)a->s_q * a->heads_q > 65536) return fail(MLA_ERR_UNSUPPORTED, "s_q * heads_q exceeds 65536");
  if (!(a->sm_scale > 0.f) || !isfinite(a->sm_scale)) return fail(MLA_ERR_INVALID, "sm_scale must be finite and > 0");
  if (!a->q_nope || !a->q_rope || !a->kv_nope || !a->kv_rope || !a->out ||
      (!a->cache_seqlens && !a->indices) || !a->tile_sched || !a->num_splits)
    return fail(MLA_ERR_INVALID, "a required pointer is NULL");
  if (!aligned(a->q_nope, 16) || !aligned(a->q_rope, 16) || !aligned(a->kv_nope, 16) ||
      !aligned(a->kv_rope, 16))
    return fail(MLA_ERR_INVALID, "q/kv pointers must be 16-byte aligned");
  const int64_t s8[] = {a->q_stride_b, a->q_stride_s, a->q_stride_h, a->q_rope_stride_b,
                        a->q_rope_stride_s, a->q_rope_stride_h, a->kv_stride_tok, a->kv_rope_stride_tok};
  for (int64_t s : s8)
    if (s < 0 || s % 8) return fail(MLA_ERR_INVALID, "q/kv strides must be non-negative multiples of 8 elements");
  // The kernel forms each lane's byte offset inside a 32-token stage in 32 bits (SGPR base
  // + 32-bit VGPR offset): 63 * stride * 2 bytes must stay far below 2^31.
  if (a->kv_stride_tok >= (int64_t(1) << 24) || a->kv_rope_stride_tok >= (int64_t(1) << 24))
    return fail(MLA_ERR_UNSUPPORTED, "kv token strides must be below 2^24 elements");
  if (a->block_table) {
    if (a->kv_stride_page < 0 || a->kv_stride_page % 8 || a->kv_rope_stride_page < 0 || a->kv_rope_stride_page % 8)
      return fail(MLA_ERR_INVALID, "page strides must be non-negative multiples of 8 elements");
    // page offsets are formed as page id (< 2^31) x 32-bit stride in 64 bits
    if (a->kv_stride_page >= (int64_t(1) << 32) || a->kv_rope_stride_page >= (int64_t(1) << 32))
      return fail(MLA_ERR_UNSUPPORTED, "page strides must be below 2^32 elements");
    if (a->block_table_stride < 1) return fail(MLA_ERR_INVALID, "block_table_stride must be >= 1");
    if (a->block_table_width < 1 || a->block_table_width > a->block_table_stride ||
        a->block_table_width > (1 << 24))
      return fail(MLA_ERR_INVALID, "block_table_width must be in [1, min(block_table_stride, 2^24)]");
    if (a->num_blocks < 1) return fail(MLA_ERR_INVALID, "num_blocks must be >= 1");
  } else {
    if (a->kv_stride_batch < 0 || a->kv_stride_batch % 8 || a->kv_rope_stride_batch < 0 ||
        a->kv_rope_stride_batch % 8)
      return fail(MLA_ERR_INVALID, "batch strides must be non-negative multiples of 8 elements");
  }
  if (!aligned(a->out, 8) || a->o_stride_b % 4 || a->o_stride_s % 4 || a->o_stride_h % 4 ||
      a->o_stride_b < 0 || a->o_stride_s < 0 || a->o_stride_h < 0)
    return fail(MLA_ERR_INVALID, "out must be 8-byte aligned with strides multiples of 4 elements");
  if (a->num_parts < 1) return fail(MLA_ERR_INVALID, "num_parts must be >= 1");
  if ((a->kv_format != MLA_KV_NATIVE && a->kv_format != MLA_KV_FP8_E4M3) || a->kv_reserved != 0)
    return fail(MLA_ERR_INVALID, "kv_format must be MLA_KV_NATIVE or MLA_KV_FP8_E4M3 (kv_reserved 0)");
  if (a->table_reserved != 0) return fail(MLA_ERR_INVALID, "table_reserved must be 0");
  if (a->status != nullptr && !aligned(a->status, 4)) return fail(MLA_ERR_INVALID, "status must be 4-byte aligned");
  if (a->indices) {
    if (a->s_q != 1) return fail(MLA_ERR_UNSUPPORTED, "the sparse decode takes s_q == 1");
    if (a->topk < 1 || a->topk > MLA_SPARSE_MAX_TOPK)
      return fail(MLA_ERR_UNSUPPORTED, "topk must be in [1, MLA_SPARSE_MAX_TOPK]");
    if (a->indices_stride < a->topk) return fail(MLA_ERR_INVALID, "indices_stride must be >= topk");
    if (a->num_blocks < 1) return fail(MLA_ERR_INVALID, "num_blocks must be >= 1");
    if (a->kv_stride_page < 0 || a->kv_stride_page % 8 || a->kv_rope_stride_page < 0 || a->kv_rope_stride_page % 8)
      return fail(MLA_ERR_INVALID, "page strides must be non-negative multiples of 8 elements");
  }
  if (a->kv_format == MLA_KV_FP8_E4M3) {
    if (a->dtype != MLA_DTYPE_BF16) return fail(MLA_ERR_UNSUPPORTED, "the fp8 cache is read with bf16 queries");
    if (!a->block_table && !a->indices) return fail(MLA_ERR_UNSUPPORTED, "the fp8 cache is paged only");
    if (a->kv_stride_page % 16 || a->kv_stride_tok % 16)
      return fail(MLA_ERR_INVALID, "fp8 latent strides must be multiples of 16 bytes");
    if (!a->kv_scale || !aligned(a->kv_scale, 16) || a->kv_scale_stride_page < 0 ||
        a->kv_scale_stride_blk < 0 || a->kv_scale_stride_page % 4 || a->kv_scale_stride_blk % 4)
      return fail(MLA_ERR_INVALID, "kv_scale must be 16-byte aligned with non-negative strides, multiples of 4 floats");
  }
  *need_ws = mla_workspace_bytes(a->batch, a->s_q, a->heads_q, a->num_parts);
  if (a->workspace == nullptr || a->workspace_bytes < *need_ws)
    return fail(MLA_ERR_WORKSPACE, "workspace missing or smaller than mla_workspace_bytes()");
  if (!aligned(a->workspace, 256)) return fail(MLA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return MLA_OK;
}

mla::KParams make_params(const mla_decode_args* a) {
  mla::KParams k{};
  k.q_nope = (const uint16_t*)a->q_nope;
  k.q_rope = (const uint16_t*)a->q_rope;
  k.q_sb = a->q_stride_b; k.q_ss = a->q_stride_s; k.q_sh = a->q_stride_h;
  k.qr_sb = a->q_rope_stride_b; k.qr_ss = a->q_rope_stride_s; k.qr_sh = a->q_rope_stride_h;
  k.kv_nope = (const uint16_t*)a->kv_nope;
  k.kv_rope = (const uint16_t*)a->kv_rope;
  k.kv_sp = a->kv_stride_page; k.kv_st = a->kv_stride_tok; k.kv_sb = a->kv_stride_batch;
  k.kr_sp = a->kv_rope_stride_page; k.kr_st = a->kv_rope_stride_tok; k.kr_sb = a->kv_rope_stride_batch;
  k.kv_scale = a->kv_format == MLA_KV_FP8_E4M3 ? a->kv_scale : nullptr;
  k.ks_sp = a->kv_scale_stride_page; k.ks_sb = a->kv_scale_stride_blk;
  k.indices = a->indices;
  k.idx_stride = a->indices_stride;
  k.topk = a->topk;
  k.pool_tokens = (int64_t)a->num_blocks * mla::kPageTokens;
  k.block_table = a->block_table;
  k.bt_stride = a->block_table_stride;
  k.bt_width = a->block_table_width;
  k.status = a->status;
  k.num_blocks = a->num_blocks;
  k.seqlens = a->cache_seqlens;
  k.sched = a->tile_sched;
  k.splits = a->num_splits;
  k.out = (uint16_t*)a->out;
  k.o_sb = a->o_stride_b; k.o_ss = a->o_stride_s; k.o_sh = a->o_stride_h;
  k.lse = a->lse;
  const int64_t rows = (int64_t)a->s_q * a->heads_q;
  const int64_t slots = (int64_t)a->batch + a->num_parts;
  k.ws_lse = (float*)a->workspace;
  k.ws_scale = (float*)((char*)a->workspace + ws_lse_bytes(slots, rows));
  k.ws_o = (uint16_t*)((char*)k.ws_scale + ws_scale_bytes(slots, rows));
  k.batch = a->batch;
  k.s_q = a->s_q;
  k.heads = a->heads_q;
  k.rows = (int)rows;
  k.causal = a->causal ? 1 : 0;
  k.num_parts = a->num_parts;
  k.scale_log2 = a->sm_scale * mla::kLog2e;
  // one cache tensor: the rope half starts 512 elements into each latent row, same strides
  k.rope_fused = (const uint16_t*)a->kv_rope == (const uint16_t*)a->kv_nope + mla::kDV &&
                 a->kv_rope_stride_tok == a->kv_stride_tok &&
                 (a->block_table ? a->kv_rope_stride_page == a->kv_stride_page
                                 : a->kv_rope_stride_batch == a->kv_stride_batch) &&
                 a->kv_format == MLA_KV_NATIVE;
  return k;
}

// Partials are the decode workspace's scaled fp16 rows (SCALED), the caller's fp32 rows of
// mla_merge_partials, or the unscaled 16-bit rows of mla_launch (PT = uint16_t).
// Many splits per sequence on average: a small grid of long merges, which the combine kernel's
// DEEP form runs with each row split in four one-wave workgroups (dim quarters).
bool combine_is_deep(const mla::KParams& k) {
  return k.num_parts >= 16 * k.batch && k.rows <= mla::kDeepMaxRows;
}

template <typename PT, bool SCALED = false>
int launch_combine(const mla::KParams& k, const PT* part_o, int dtype, int copy_single, hipStream_t st) {
  const bool deep = std::is_same<PT, uint16_t>::value && combine_is_deep(k);
  const int W = deep ? 1 : 4;
  const dim3 grid(k.batch, (k.rows + W - 1) / W, deep ? 4 : 1);
#define MLA_COMBINE(D, DP)                                                                                      \
  hipLaunchKernelGGL((mla::mla_combine_kernel<D, PT, SCALED, DP>), grid, dim3(64 * W), 0, st, part_o, k.ws_scale, \
                     k.ws_lse, k.splits, k.rows, k.heads, k.s_q, k.out, k.o_sb, k.o_ss, k.o_sh, k.lse, copy_single)
  if (dtype == MLA_DTYPE_BF16) {
    if (deep) MLA_COMBINE(MLA_DTYPE_BF16, true); else MLA_COMBINE(MLA_DTYPE_BF16, false);
  } else {
    if (deep) MLA_COMBINE(MLA_DTYPE_F16, true); else MLA_COMBINE(MLA_DTYPE_F16, false);
  }
#undef MLA_COMBINE
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MLA_ERR_HIP, std::string("combine launch failed: ") + hipGetErrorString(e));
  return MLA_OK;
}

}  // namespace

extern "C" {

int mla_version(void) { return MLA_DECODE_AMD_VERSION; }

const char* mla_last_error(void) { return g_last_error.c_str(); }

int mla_variant(int32_t rows, int32_t* waves, int32_t* row_tiles, int32_t* stages,
                int32_t* rows_per_workgroup) {
  if (rows < 1 || !waves || !row_tiles || !stages || !rows_per_workgroup)
    return fail(MLA_ERR_INVALID, "rows must be >= 1 and outputs non-NULL");
  const Variant v = pick_variant(rows);
  *waves = v.nw;
  *row_tiles = v.ht;
  *stages = (!v.ws && v.nw == 4 && wide_enabled()) ? mla::kWideLat : v.nstage;  // the wide kernel's ring
  *rows_per_workgroup = v.rows();
  return MLA_OK;
}

int mla_num_parts(int32_t batch, int32_t s_q, int32_t heads_q, int32_t heads_k, int32_t cu_count) {
  if (batch < 1 || s_q < 1 || heads_q < 1 || heads_k != 1) {
    fail(MLA_ERR_INVALID, "invalid shape");
    return -MLA_ERR_INVALID;
  }
  const int rows = s_q * heads_q;
  const Variant v = pick_variant(rows);
  const int R = v.rows();
  const int head_blocks = (rows + R - 1) / R;
  const int cus = cu_count > 0 ? cu_count : cu_count_current();
  int parts = cus * wgs_per_cu(v) / head_blocks;
  return parts < 1 ? 1 : parts;
}

int mla_get_metadata_host(const int32_t* cache_seqlens, int32_t batch, int32_t num_parts,
                          int32_t fixed_overhead, int32_t forced_splits, int32_t* tile_sched,
                          int32_t* num_splits) {
  if (!cache_seqlens || !tile_sched || !num_splits) return fail(MLA_ERR_INVALID, "NULL pointer");
  if (batch < 1) return fail(MLA_ERR_INVALID, "batch must be >= 1");
  if (forced_splits > 0) {
    if ((int64_t)num_parts != (int64_t)batch * forced_splits)
      return fail(MLA_ERR_INVALID, "forced_splits requires num_parts == batch * forced_splits");
    mla::schedule_forced(cache_seqlens, batch, forced_splits, tile_sched, num_splits);
  } else {
    if (num_parts < 1) return fail(MLA_ERR_INVALID, "num_parts must be >= 1");
    std::vector<int32_t> pages(batch);
    mla::schedule_packed(cache_seqlens, batch, num_parts,
                         fixed_overhead < 0 ? mla::kDefaultSplitOverhead : fixed_overhead,
                         fixed_overhead < 0, pages.data(), tile_sched, num_splits);
  }
  return MLA_OK;
}

int mla_get_metadata(const int32_t* cache_seqlens, int32_t batch, int32_t num_parts,
                     int32_t fixed_overhead, int32_t forced_splits, int32_t* tile_sched,
                     int32_t* num_splits, void* stream) {
  if (!cache_seqlens || !tile_sched || !num_splits) return fail(MLA_ERR_INVALID, "NULL pointer");
  if (batch < 1 || batch > mla::kMetaMaxBatch) return fail(MLA_ERR_INVALID, "batch must be in [1, 16384]");
  if (forced_splits > 0) {
    if ((int64_t)num_parts != (int64_t)batch * forced_splits)
      return fail(MLA_ERR_INVALID, "forced_splits requires num_parts == batch * forced_splits");
  } else if (num_parts < 1) {
    return fail(MLA_ERR_INVALID, "num_parts must be >= 1");
  }
  // min-payload candidates: kDefaultSplitOverhead + 1 <= kMetaMaxCand (static_assert)
  hipLaunchKernelGGL(mla::mla_metadata_kernel, dim3(1), dim3(mla::kMetaThreads), 0,
                     (hipStream_t)stream, cache_seqlens, batch, num_parts,
                     fixed_overhead < 0 ? mla::kDefaultSplitOverhead : fixed_overhead,
                     fixed_overhead < 0 ? 1 : 0, forced_splits, tile_sched, num_splits);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MLA_ERR_HIP, std::string("metadata launch failed: ") + hipGetErrorString(e));
  return MLA_OK;
}

int64_t mla_workspace_bytes(int32_t batch, int32_t s_q, int32_t heads_q, int32_t num_parts) {
  if (batch < 1 || s_q < 1 || heads_q < 1 || num_parts < 1) return 0;
  const int64_t rows = (int64_t)s_q * heads_q;
  const int64_t slots = (int64_t)batch + num_parts;
  return ws_lse_bytes(slots, rows) + ws_scale_bytes(slots, rows) + slots * rows * mla::kDV * 2;
}

int mla_decode_fwd(const mla_decode_args* args, void* stream) {
  const int rc = mla_splitkv_fwd(args, stream);
  if (rc != MLA_OK) return rc;
  const mla::KParams kp = make_params(args);
  return launch_combine<uint16_t, true>(kp, kp.ws_o, args->dtype, 0, (hipStream_t)stream);
}

// The allocation-free decode's scratch: one array per GPU (each device that loads this code
// object holds its own copy), addressed from the host only through the pointer that
// hipGetSymbolAddress returns for that device.
static __device__ __align__(256) uint8_t scratch[MLA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up once per device (with that device current).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MLA_ERR_HIP, std::string("hipGetDevice failed: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MLA_ERR_UNSUPPORTED, "device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(MLA_ERR_HIP, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MLA_OK;
}
}  // namespace

int mla_decode_fwd_noalloc(const mla_decode_args* args, void* stream) {
  if (!args) return fail(MLA_ERR_INVALID, "args is NULL");
  if (args->workspace != nullptr || args->workspace_bytes != 0)
    return fail(MLA_ERR_INVALID, "mla_decode_fwd_noalloc takes no workspace (workspace NULL, workspace_bytes 0)");
  const int64_t need = mla_workspace_bytes(args->batch, args->s_q, args->heads_q, args->num_parts);
  if (need > MLA_NOALLOC_SCRATCH_BYTES)
    return fail(MLA_ERR_WORKSPACE, "problem needs " + std::to_string(need) +
                                       " workspace bytes, more than MLA_NOALLOC_SCRATCH_BYTES");
  mla_decode_args a = *args;
  const int rc = scratch_address(&a.workspace);
  if (rc != MLA_OK) return rc;
  a.workspace_bytes = MLA_NOALLOC_SCRATCH_BYTES;
  return mla_decode_fwd(&a, stream);
}

int mla_splitkv_fwd(const mla_decode_args* args, void* stream) {
  int64_t need = 0;
  const int rc = validate(args, &need);
  if (rc != MLA_OK) return rc;
  const mla::KParams kp = make_params(args);
  const Variant v = pick_variant(kp.rows);
  const int R = v.rows();
  const int head_blocks = (kp.rows + R - 1) / R;
  const hipError_t e = args->dtype == MLA_DTYPE_BF16
                           ? launch_main_dt<MLA_DTYPE_BF16>(v, kp, head_blocks, (hipStream_t)stream)
                           : launch_main_dt<MLA_DTYPE_F16>(v, kp, head_blocks, (hipStream_t)stream);
  if (e != hipSuccess) return fail(MLA_ERR_HIP, std::string("decode launch failed: ") + hipGetErrorString(e));
  return MLA_OK;
}

int mla_combine_fwd(const mla_decode_args* args, void* stream) {
  int64_t need = 0;
  const int rc = validate(args, &need);
  if (rc != MLA_OK) return rc;
  const mla::KParams kp = make_params(args);
  return launch_combine<uint16_t, true>(kp, kp.ws_o, args->dtype, 0, (hipStream_t)stream);
}

int mla_combine_absorb(const mla_decode_args* args, const void* w_uv_blk, void* v, void* stream) {
  int64_t need = 0;
  const int rc = validate(args, &need);
  if (rc != MLA_OK) return rc;
  if (!w_uv_blk || !v) return fail(MLA_ERR_INVALID, "w_uv_blk and v must not be NULL");
  if (!aligned(w_uv_blk, 16)) return fail(MLA_ERR_INVALID, "w_uv_blk must be 16-byte aligned");
  if (!aligned(v, 4)) return fail(MLA_ERR_INVALID, "v must be 4-byte aligned");
  const mla::KParams kp = make_params(args);
  mla::AbsorbParams a{};
  a.ws_o = kp.ws_o;
  a.ws_scale = kp.ws_scale;
  a.ws_lse = kp.ws_lse;
  a.splits = kp.splits;
  a.out = kp.out;
  a.o_sb = kp.o_sb; a.o_ss = kp.o_ss; a.o_sh = kp.o_sh;
  a.w_blk = (const uint16_t*)w_uv_blk;
  a.v = (uint16_t*)v;
  a.lse = kp.lse;
  a.m_rows = kp.batch * kp.s_q;
  a.s_q = kp.s_q;
  a.heads = kp.heads;
  a.rows = kp.rows;
  if (combine_is_deep(kp)) {
    // long merges: the combine kernel's DEEP form writes the merged rows (bf16/fp16, as the
    // fused merge rounds them into LDS) and their lse, and the projection reads every row from
    // `out`; v is bit-identical to the fused merge's
    const int rc2 = launch_combine<uint16_t, true>(kp, kp.ws_o, args->dtype, 0, (hipStream_t)stream);
    if (rc2 != MLA_OK) return rc2;
    a.premerged = 1;
  }
  const dim3 grid(kp.heads, (a.m_rows + mla::kAbsRows - 1) / mla::kAbsRows);
  if (args->dtype == MLA_DTYPE_BF16)
    hipLaunchKernelGGL(mla::mla_combine_absorb_kernel<MLA_DTYPE_BF16>, grid, dim3(256), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(mla::mla_combine_absorb_kernel<MLA_DTYPE_F16>, grid, dim3(256), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MLA_ERR_HIP, std::string("combine-absorb launch failed: ") + hipGetErrorString(e));
  return MLA_OK;
}

int mla_merge_partials(const float* part_o, const float* part_lse, const int32_t* num_splits,
                       int32_t batch, int32_t rows, int32_t dtype, void* out, float* lse_out,
                       void* stream) {
  if (!part_o || !part_lse || !num_splits || !out) return fail(MLA_ERR_INVALID, "NULL pointer");
  if (batch < 1 || rows < 1) return fail(MLA_ERR_INVALID, "batch and rows must be >= 1");
  if (dtype != MLA_DTYPE_BF16 && dtype != MLA_DTYPE_F16) return fail(MLA_ERR_INVALID, "bad dtype");
  if (!aligned(part_o, 16) || !aligned(out, 16)) return fail(MLA_ERR_INVALID, "part_o and out must be 16-byte aligned");
  mla::KParams k{};
  k.ws_lse = (float*)part_lse;
  k.splits = num_splits;
  k.batch = batch;
  k.rows = rows;
  k.heads = rows;
  k.s_q = 1;
  k.out = (uint16_t*)out;
  k.o_sb = (int64_t)rows * mla::kDV;
  k.o_ss = 0;
  k.o_sh = mla::kDV;
  k.lse = lse_out;
  return launch_combine(k, part_o, dtype, 1, (hipStream_t)stream);
}

int mla_split_plan(int32_t seqlen_kv, int32_t num_split, int32_t block_n, int32_t spread,
                   int32_t* ns_out, int32_t* blocks_per_split_out, int32_t* extra_out) {
  if (seqlen_kv < 1 || num_split < 1 || block_n < 1 || !ns_out || !blocks_per_split_out || !extra_out)
    return fail(MLA_ERR_INVALID, "seqlen_kv, num_split and block_n must be >= 1");
  const int nb = (seqlen_kv + block_n - 1) / block_n;
  if (!spread) {
    const int chunk = (seqlen_kv + num_split - 1) / num_split;
    int bpc = (chunk + block_n - 1) / block_n;
    if (bpc < 1) bpc = 1;
    int ns = (nb + bpc - 1) / bpc;
    if (ns < 1) ns = 1;
    *ns_out = ns;
    *blocks_per_split_out = bpc;
    *extra_out = 0;
  } else {
    int ns = num_split < nb ? num_split : nb;
    if (ns < 1) ns = 1;
    *ns_out = ns;
    *blocks_per_split_out = nb / ns;
    *extra_out = nb % ns;
  }
  return MLA_OK;
}

void mla_launch(const void* Q, const void* Qpe, const void* KV, const void* Kpe, void* glse,
                void* partial, void* out, int ns) {
  // The reference's frozen shape: B = 1, H = 16, L = 8192, fp16, contiguous [B, L, 1, D] cache,
  // sm_scale = 576^-0.5, launched on the null stream.  Caller scratch: glse (fp16
  // [1, 16, ns + 64]: 32 * (ns + 64) bytes) holds the sequence length, the split prefix sums
  // and the ns-part tile schedule; partial (fp16 [1, 16, ns, 576]: 18432 * ns bytes) holds the
  // per-split lse (fp32, padded to 256 bytes) and the 16-bit partial rows [ns, 16, 512].
  constexpr int kPages = mla::kHandCtx / mla::kPageTokens;
  if (!Q || !Qpe || !KV || !Kpe || !glse || !partial || !out) {
    fail(MLA_ERR_INVALID, "mla_launch: a pointer is NULL");
    return;
  }
  if (ns < 1 || ns > kPages) {
    fail(MLA_ERR_INVALID, "mla_launch: ns must be in [1, 128] (the 8192-token cache has 128 pages)");
    return;
  }
  if (!aligned(Q, 16) || !aligned(Qpe, 16) || !aligned(KV, 16) || !aligned(Kpe, 16) || !aligned(glse, 16) ||
      !aligned(partial, 16) || !aligned(out, 16)) {
    fail(MLA_ERR_INVALID, "mla_launch: every buffer must be 16-byte aligned");
    return;
  }
  char* g = (char*)glse;
  int32_t* seqlens = (int32_t*)g;          // [1]
  int32_t* splits = (int32_t*)(g + 16);    // [2]
  int32_t* sched = (int32_t*)(g + 64);     // [ns, 8]: 64 + 32 ns <= 32 (ns + 64) bytes
  const int64_t lse_bytes = ws_lse_bytes(ns, mla::kHandHeads);  // <= 64 ns + 255
  mla::KParams k{};
  k.q_nope = (const uint16_t*)Q;
  k.q_rope = (const uint16_t*)Qpe;
  k.q_sb = mla::kHandHeads * 512; k.q_ss = 0; k.q_sh = 512;
  k.qr_sb = mla::kHandHeads * 64; k.qr_ss = 0; k.qr_sh = 64;
  k.kv_nope = (const uint16_t*)KV;
  k.kv_rope = (const uint16_t*)Kpe;
  k.kv_st = 512; k.kv_sb = (int64_t)mla::kHandCtx * 512;
  k.kr_st = 64; k.kr_sb = (int64_t)mla::kHandCtx * 64;
  k.block_table = nullptr;
  k.num_blocks = 1;
  k.seqlens = seqlens;
  k.sched = sched;
  k.splits = splits;
  k.out = (uint16_t*)out;
  k.o_sb = mla::kHandHeads * 512; k.o_ss = 0; k.o_sh = 512;
  k.lse = nullptr;
  // lse_bytes + 16 * 512 * 2 * ns <= 18432 ns bytes for every ns >= 1
  k.ws_lse = (float*)partial;
  k.ws_o = (uint16_t*)((char*)partial + lse_bytes);
  k.part16 = 1;
  k.batch = 1;
  k.s_q = 1;
  k.heads = mla::kHandHeads;
  k.rows = mla::kHandHeads;
  k.causal = 0;
  k.num_parts = ns;
  k.scale_log2 = mla::kLog2e / sqrtf((float)MLA_DIM_QK);
  hipStream_t st = nullptr;
  hipLaunchKernelGGL(mla::mla_launch_sched_kernel, dim3(1), dim3(64), 0, st, seqlens, sched, splits, ns);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = launch_main_dt<MLA_DTYPE_F16>(pick_variant(k.rows), k, 1, st);
  if (e != hipSuccess) {
    fail(MLA_ERR_HIP, std::string("mla_launch: launch failed: ") + hipGetErrorString(e));
    return;
  }
  launch_combine(k, (const uint16_t*)k.ws_o, MLA_DTYPE_F16, 0, st);  // unscaled 16-bit rows
}

int mla_kv_append(const mla_kv_append_args* a, void* stream) {
  if (a == nullptr) return fail(MLA_ERR_INVALID, "args is NULL");
  if (a->batch < 1 || a->n_new < 1 || a->n_new > mla::kPageTokens)
    return fail(MLA_ERR_INVALID, "batch must be >= 1 and n_new in [1, 64]");
  if (a->dtype != MLA_DTYPE_BF16 && a->dtype != MLA_DTYPE_F16)
    return fail(MLA_ERR_INVALID, "dtype must be MLA_DTYPE_BF16 or MLA_DTYPE_F16");
  if (!a->kv_new || !a->kv_nope || !a->kv_rope || !a->block_table || !a->cache_seqlens)
    return fail(MLA_ERR_INVALID, "a required pointer is NULL");
  if (!aligned(a->kv_new, 16) || !aligned(a->kv_nope, 16) || !aligned(a->kv_rope, 16))
    return fail(MLA_ERR_INVALID, "kv_new / cache pointers must be 16-byte aligned");
  const int64_t s8[] = {a->new_stride_b, a->new_stride_t, a->kv_stride_page, a->kv_stride_tok,
                        a->kv_rope_stride_page, a->kv_rope_stride_tok};
  for (int64_t v : s8)
    if (v < 0 || v % 8) return fail(MLA_ERR_INVALID, "strides must be non-negative multiples of 8 elements");
  if (a->block_table_stride < 1 || a->max_pages < 1 || a->num_blocks < 1)
    return fail(MLA_ERR_INVALID, "block_table_stride, max_pages and num_blocks must be >= 1");
  if ((a->kv_format != MLA_KV_NATIVE && a->kv_format != MLA_KV_FP8_E4M3) || a->kv_reserved != 0)
    return fail(MLA_ERR_INVALID, "kv_format must be MLA_KV_NATIVE or MLA_KV_FP8_E4M3 (kv_reserved 0)");
  const bool kv8 = a->kv_format == MLA_KV_FP8_E4M3;
  if (kv8) {
    if (a->dtype != MLA_DTYPE_BF16) return fail(MLA_ERR_UNSUPPORTED, "the fp8 cache takes bf16 tokens");
    if (a->kv_stride_page % 16 || a->kv_stride_tok % 16)
      return fail(MLA_ERR_INVALID, "fp8 latent strides must be multiples of 16 bytes");
    if (!a->kv_scale || !aligned(a->kv_scale, 16) || a->kv_scale_stride_page < 0 ||
        a->kv_scale_stride_blk < 0 || a->kv_scale_stride_page % 4 || a->kv_scale_stride_blk % 4)
      return fail(MLA_ERR_INVALID, "kv_scale must be 16-byte aligned with non-negative strides, multiples of 4 floats");
  }
  mla::AppendParams k{};
  k.kv_new = (const uint16_t*)a->kv_new;
  k.n_sb = a->new_stride_b; k.n_st = a->new_stride_t;
  k.kv_nope = (uint16_t*)a->kv_nope; k.kv_rope = (uint16_t*)a->kv_rope;
  k.kv_sp = a->kv_stride_page; k.kv_st = a->kv_stride_tok;
  k.kr_sp = a->kv_rope_stride_page; k.kr_st = a->kv_rope_stride_tok;
  k.block_table = a->block_table;
  k.bt_stride = a->block_table_stride; k.max_pages = a->max_pages; k.num_blocks = a->num_blocks;
  k.batch = a->batch; k.n_new = a->n_new;
  k.seqlens = a->cache_seqlens;
  k.status = a->status;
  k.kv8 = kv8 ? 1 : 0;
  k.kv_scale = a->kv_scale;
  k.ks_sp = a->kv_scale_stride_page; k.ks_sb = a->kv_scale_stride_blk;
  hipLaunchKernelGGL(mla::mla_kv_append_kernel, dim3((a->batch + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MLA_ERR_HIP, std::string("kv append launch failed: ") + hipGetErrorString(e));
  return MLA_OK;
}

}  // extern "C"
#endif  // MLA_WS_TU
