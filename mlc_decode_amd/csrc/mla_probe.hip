// mla_probe.hip -- measurement helper for bench.py (not part of the decode library's ABI):
// the dense bf16 MFMA rate the device sustains and its shader clock under that load, the
// denominators of the MFMA-bound configurations' measured-peak fractions (as the stream probe
// in bench.py measures the achievable HBM rate).
//
//   extern "C" int mla_probe_mfma(int iters, float* sink, unsigned long long* clocks,
//                                 int workgroups, void* stream)
//
// launches `workgroups` workgroups of four waves; each wave runs `iters` rounds of eight
// independent v_mfma_f32_16x16x32_bf16 chains (8 * 16384 flops per round) and stores its
// accumulators into sink[workgroups * 256 * 4]; lane 0 of wave 0 of workgroup w writes
// clocks[4w .. 4w+3] = {shader clock at start, wall clock at start, shader clock at end,
// wall clock at end} (clock64 / wall_clock64).  Returns 0 or the HIP error code.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));

__global__ __launch_bounds__(256, 2) void mfma_rate_kernel(int iters, float* sink, unsigned long long* clocks) {
  const int lane = threadIdx.x & 63;
  const bool lead = threadIdx.x == 0;
  unsigned long long c0 = 0, w0 = 0;
  if (lead) {
    c0 = clock64();
    w0 = wall_clock64();
  }
  // operands that depend on the lane, so nothing folds to a constant
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.001f * (float)(lane + i));
    b[i] = (__bf16)(0.002f * (float)(lane - i));
  }
  f32x4 acc[8];
  for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
  }
  f32x4 s = acc[0];
  for (int c = 1; c < 8; ++c) s += acc[c];
  *(f32x4*)(sink + ((size_t)blockIdx.x * 256 + threadIdx.x) * 4) = s;
  if (lead) {
    const unsigned long long c1 = clock64();
    const unsigned long long w1 = wall_clock64();
    unsigned long long* o = clocks + (size_t)blockIdx.x * 4;
    o[0] = c0;
    o[1] = w0;
    o[2] = c1;
    o[3] = w1;
  }
}

}  // namespace

extern "C" int mla_probe_mfma(int iters, float* sink, unsigned long long* clocks, int workgroups, void* stream) {
  if (iters < 1 || workgroups < 1 || sink == nullptr || clocks == nullptr) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_rate_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream, iters, sink, clocks);
  return (int)hipGetLastError();
}

// Frequency of wall_clock64() in kHz (hipDeviceAttributeWallClockRate), or a negative error.
extern "C" int mla_probe_wall_clock_khz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return -1;
  return khz;
}
