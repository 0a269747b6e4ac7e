/*
 * mla_decode_amd.h -- C ABI of the MI355X (gfx950) MLA decode library.
 *
 * Multi-head latent attention decode against one shared latent KV head:
 *   q        [B, s_q, H, 576]   (512 latent "nope" dims + 64 rope dims)
 *   kv cache [num_blocks, 64, 1, 576] paged, V = the first 512 dims of K
 *   out      [B, s_q, H, 512],  lse [B, H, s_q] fp32 (natural log)
 *
 * Every buffer is caller-owned device memory; every entry point takes an
 * explicit stream and returns 0 on success or a nonzero MLA_ERR_* code, with
 * a message readable through mla_last_error() on the calling thread.  Nothing
 * here allocates device memory: the split-KV workspace is sized by
 * mla_workspace_bytes() and passed in.
 *
 * Reference interfaces each entry point replaces (paths are relative to the
 * reference repository NiseAzaka/mlc_decode):
 *   - mla_launch            handmade/mla_handmade.py:34-52 (extern "C" mla_launch)
 *   - mla_get_metadata      the get_mla_metadata call of handmade/bench_metax_flashmla.py:31
 *                           (algorithm described in docs/num_split_design.md:31-135)
 *   - mla_decode_fwd        the flash_mla_with_kvcache call of handmade/bench_metax_flashmla.py:33-35,
 *                           and the main + combine TileLang kernels of mla_decode.py:78-259
 *   - mla_splitkv_fwd       the main split-KV TileLang kernel alone, mla_decode.py:78-192
 *   - mla_combine_fwd       the combine kernel of mla_decode.py:194-246 (LSE-weighted merge)
 *   - mla_split_plan        _split_plan of mla_decode.py:9-30
 */
#ifndef MLA_DECODE_AMD_H
#define MLA_DECODE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: mla_decode_args gained block_table_width / table_reserved / status (a decode bounded by
 * the block table's width). */
#define MLA_DECODE_AMD_VERSION 2

/* dtypes of q / kv / out */
#define MLA_DTYPE_BF16 0
#define MLA_DTYPE_F16 1

/* status codes */
#define MLA_OK 0
#define MLA_ERR_INVALID 1   /* bad shape, stride, pointer alignment or dtype */
#define MLA_ERR_WORKSPACE 2 /* workspace missing or too small */
#define MLA_ERR_HIP 3       /* a HIP runtime call failed (launch error etc.) */
#define MLA_ERR_UNSUPPORTED 4

/* Fixed geometry of the latent cache. */
#define MLA_DIM_QK 576
#define MLA_DIM_V 512
#define MLA_PAGE_TOKENS 64
/* Each part of the tile schedule is described by this many int32 words. */
#define MLA_SCHED_WORDS 8
/* Per-split overhead, in pages, of the default (min-payload) tile schedule. */
#define MLA_DEFAULT_SPLIT_OVERHEAD 3

/* Longest top-k index list of the sparse decode. */
#define MLA_SPARSE_MAX_TOPK 2048

/* KV cache formats (mla_decode_args.kv_format, mla_kv_append_args.kv_format). */
#define MLA_KV_NATIVE 0   /* latent and rope in the query dtype */
#define MLA_KV_FP8_E4M3 1 /* latent as OCP e4m3 codes with power-of-two scales (below) */

/*
 * Decode arguments.  Strides are in elements.  The latent ("nope", dims
 * 0..511) and rope (dims 512..575) halves may live in one tensor (rope pointer
 * = latent pointer + 512, same strides) or in two tensors.
 *
 * KV addressing:
 *   block_table != NULL (paged):  token t of sequence b lives in page
 *     p = block_table[b * block_table_stride + t / 64], row t % 64 (t / 64 below
 *     block_table_width; tokens past 64 * block_table_width are not read, see below):
 *     latent at kv_nope + p*kv_stride_page + (t%64)*kv_stride_tok
 *     rope   at kv_rope + p*kv_rope_stride_page + (t%64)*kv_rope_stride_tok
 *   block_table == NULL (contiguous, the reference's [B, L, 1, D] layout):
 *     latent at kv_nope + b*kv_stride_batch + t*kv_stride_tok (rope alike).
 * q element (b, s, h, d) is at q_nope + b*q_stride_b + s*q_stride_s + h*q_stride_h + d
 * (d < 512) or q_rope + b*q_rope_stride_b + s*q_rope_stride_s + h*q_rope_stride_h + (d - 512).
 * lse may be NULL (not written).
 * Alignment: q/kv base pointers 16-byte aligned and their strides multiples of 8 elements;
 * out 8-byte aligned with strides multiples of 4; workspace 256-byte aligned.
 * out element (b, s, h, d) is at out + b*o_stride_b + s*o_stride_s + h*o_stride_h + d.
 * lse is a contiguous fp32 [B, H, s_q] array (natural log of the softmax denominator
 * of sm_scale * q.k); rows with no visible key get out = 0 and lse = -inf.
 *
 * kv_format == MLA_KV_FP8_E4M3 (paged or sparse, dtype bf16): kv_nope points to uint8 OCP e4m3
 * codes (strides in bytes: 16-byte multiples; a token's 512 codes contiguous); kv_rope holds
 * the rope dims in bf16 as above; kv_scale holds fp32 scales, the scale of token row r of
 * page p and 128-dim block j (dims 128j .. 128j+127) at
 *   kv_scale + p*kv_scale_stride_page + j*kv_scale_stride_blk + r
 * (strides in floats, multiples of 4, pointer 16-byte aligned).  Latent value d of a token is
 * e4m3(code_d) * scale_{d/128}; every scale must be a power of two (2^-126 .. 2^127), as
 * mla_kv_append writes them: the device applies it as an exponent.  The rope and the
 * queries are bf16.  With MLA_KV_NATIVE, kv_scale is unused and may be NULL.
 */
typedef struct mla_decode_args {
  int32_t batch;
  int32_t s_q;
  int32_t heads_q;
  int32_t heads_k; /* must be 1 (one shared latent head) */
  int32_t dtype;   /* MLA_DTYPE_BF16 or MLA_DTYPE_F16 */
  int32_t causal;  /* s_q > 1: query i sees keys [0, L - s_q + i] */
  float sm_scale;
  int32_t num_blocks; /* pool size of the paged cache (page ids are clamped to it) */

  const void* q_nope;
  const void* q_rope;
  int64_t q_stride_b, q_stride_s, q_stride_h;
  int64_t q_rope_stride_b, q_rope_stride_s, q_rope_stride_h;

  const void* kv_nope;
  const void* kv_rope;
  int64_t kv_stride_page, kv_stride_tok, kv_stride_batch;
  int64_t kv_rope_stride_page, kv_rope_stride_tok, kv_rope_stride_batch;

  const int32_t* block_table; /* [B, block_table_stride] int32 or NULL */
  int32_t block_table_stride;
  int32_t num_parts;            /* rows of tile_sched */
  const int32_t* cache_seqlens; /* [B] int32 (device) */
  const int32_t* tile_sched;    /* [num_parts, MLA_SCHED_WORDS] from mla_get_metadata */
  const int32_t* num_splits;    /* [B + 1] prefix sums from mla_get_metadata */

  void* out;
  int64_t o_stride_b, o_stride_s, o_stride_h;
  float* lse;

  void* workspace;
  int64_t workspace_bytes;

  int32_t kv_format;   /* MLA_KV_NATIVE or MLA_KV_FP8_E4M3 */
  int32_t kv_reserved; /* must be 0 */
  const float* kv_scale;
  int64_t kv_scale_stride_page, kv_scale_stride_blk;

  /* Sparse (top-k) decode when indices != NULL (s_q == 1, either cache format): the keys of
   * sequence b are the pool tokens indices[b * indices_stride + j], j < topk
   * (1 .. MLA_SPARSE_MAX_TOPK), token id = page * 64 + row of the paged cache (kv_nope /
   * kv_rope / kv_scale with the page strides);
   * an index < 0 or >= num_blocks * 64 names no key.  block_table and cache_seqlens are not
   * read; the schedule (tile_sched / num_splits) must be the one mla_get_metadata gives for
   * sequence lengths all equal to topk. */
  const int32_t* indices;
  int32_t indices_stride;
  int32_t topk;

  /* Paged mode: the number of valid columns of block_table (1 .. block_table_stride, at most
   * 2^24).  A sequence needs pages_of(L) = ceil(L / 64) columns; a sequence whose
   * cache_seqlens entry exceeds 64 * block_table_width is decoded over its first
   * 64 * block_table_width tokens only, no column at or past the width is read, and *status is
   * set to 1 (when status is non-NULL; the caller clears it).  Unused in contiguous and
   * sparse mode. */
  int32_t block_table_width;
  int32_t table_reserved; /* must be 0 */
  int32_t* status;        /* optional device int32, set to 1 on a length past the table */
} mla_decode_args;

/* Library version (MLA_DECODE_AMD_VERSION). */
int mla_version(void);

/* Message for the last nonzero status returned on this thread ("" if none). */
const char* mla_last_error(void);

/*
 * Number of schedule parts the decode kernel is laid out for on a device with
 * cu_count compute units (cu_count <= 0: query the current device).
 * Replaces the num_sm_parts rule described in docs/num_split_design.md:53-71.
 */
int mla_num_parts(int32_t batch, int32_t s_q, int32_t heads_q, int32_t heads_k, int32_t cu_count);

/*
 * Kernel tile chosen for `rows` = s_q * heads_q query rows (dense bf16/fp16 cache): waves per
 * workgroup, 16-row tiles per wave (of the QK product), LDS stages of 32 tokens resident per
 * ring, rows per workgroup.  Above 32 rows this is the wide kernel (PV split by output dims
 * across the waves, a 4-stage latent ring); when rows_per_workgroup is 16 * row_tiles (less
 * than waves * 16 * row_tiles), the waves share one row tile and take turns over the KV
 * stages, each with its own one-stage ring, and merge their results at the end of every
 * segment.  Returns 0, or
 * MLA_ERR_INVALID for rows < 1 or a NULL output.  Replaces the block_H / threads / stages
 * fields of the tuned-config record (mla_best_configs.json:1-73).
 */
int mla_variant(int32_t rows, int32_t* waves, int32_t* row_tiles, int32_t* stages,
                int32_t* rows_per_workgroup);

/*
 * Tile schedule on the device (one tiny kernel on `stream`).
 * cache_seqlens: [B] int32; tile_sched: [num_parts, 8] int32 out; num_splits: [B+1] int32 out.
 * forced_splits <= 0: greedy packing over num_parts parts in (sequence, page) order, a split
 *   costing its 64-token pages plus a per-split overhead of f pages, up to a payload per part:
 *   fixed_overhead >= 0: f = fixed_overhead and the reference's payload
 *     ceil(total / num_parts) + f, total = sum of (pages + f) (FlashMLA's rule);
 *   fixed_overhead < 0: f = MLA_DEFAULT_SPLIT_OVERHEAD and the smallest payload in
 *     [ceil(total / num_parts), ceil(total / num_parts) + f] whose packing fits num_parts parts
 *     (the default: the shortest critical part the greedy rule allows).
 * forced_splits > 0: every sequence is cut into min(forced_splits, pages) contiguous
 *   near-equal page ranges (the spread family of mla_decode.py:9-30); then
 *   num_parts must equal batch * forced_splits.
 * Replaces get_mla_metadata (handmade/bench_metax_flashmla.py:31).
 */
int mla_get_metadata(const int32_t* cache_seqlens, int32_t batch, int32_t num_parts,
                     int32_t fixed_overhead, int32_t forced_splits, int32_t* tile_sched,
                     int32_t* num_splits, void* stream);

/* The same schedule computed on the host from host arrays (no GPU needed). */
int mla_get_metadata_host(const int32_t* cache_seqlens, int32_t batch, int32_t num_parts,
                          int32_t fixed_overhead, int32_t forced_splits, int32_t* tile_sched,
                          int32_t* num_splits);

/*
 * Workspace bytes mla_decode_fwd needs for this problem and part count: the per-split
 * log2-domain lse [slots, rows] fp32, then the scales [slots, rows, 4] fp32, then the
 * per-split softmax-normalised partial outputs [slots, rows, 512] fp16 (each region padded to
 * 256 bytes), with slots = batch + num_parts.  Chunk c (dims 128c .. 128c+127) of a partial row
 * is stored times 2^e, e chosen from the chunk's amax so that it lands in [2^14, 2^15); the
 * scale entry holds 2^-e.  Every value is then kept to 2^-11 of its chunk's amax.  (The
 * reference's output_partial is unscaled in the input dtype, mla_decode.py:73-74; for bf16 a
 * second bf16 rounding moves outputs in [2, 4) past 1e-2, which scaled fp16 does not.)
 */
int64_t mla_workspace_bytes(int32_t batch, int32_t s_q, int32_t heads_q, int32_t num_parts);

/*
 * Split-KV decode: main kernel (one workgroup per (schedule part, head block))
 * followed by the LSE combine for sequences cut into more than one split.
 * Replaces flash_mla_with_kvcache (handmade/bench_metax_flashmla.py:33-35) and the
 * TileLang main + combine kernels (mla_decode.py:78-259).
 */
int mla_decode_fwd(const mla_decode_args* args, void* stream);

/*
 * mla_decode_fwd without a workspace and without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The split partials and LSEs go to a static device
 * array of MLA_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until the process
 * ends; args->workspace must be NULL and args->workspace_bytes 0.  A problem whose
 * mla_workspace_bytes() exceeds MLA_NOALLOC_SCRATCH_BYTES is rejected with MLA_ERR_WORKSPACE
 * before anything is launched.  Every call on one GPU uses that GPU's one array: calls that
 * overlap on a GPU (other streams, other host threads) race, and the caller must order them.
 * The same kernels and results as mla_decode_fwd.
 */
#define MLA_NOALLOC_SCRATCH_BYTES (160ll << 20)
int mla_decode_fwd_noalloc(const mla_decode_args* args, void* stream);

/*
 * Main split-KV kernel alone (the first half of mla_decode_fwd): sequences with a single
 * split are finished (out, lse); the partials of split sequences are left in `workspace`
 * for mla_combine_fwd.  Replaces the main TileLang kernel of mla_decode.py:78-192.
 */
int mla_splitkv_fwd(const mla_decode_args* args, void* stream);

/*
 * Combine stage alone, over partials produced by mla_decode_fwd into `workspace`
 * (run by mla_decode_fwd itself; exposed for testing and for callers that fuse
 * the split and merge differently).  Replaces mla_decode.py:194-246.
 */
int mla_combine_fwd(const mla_decode_args* args, void* stream);

/*
 * Stand-alone LSE merge of explicit partials: for each (b, row) with
 * n = num_splits[b+1] - num_splits[b] splits at slots num_splits[b] .. +n-1:
 *   part_o  [slots, rows, 512] fp32 (each split's softmax-normalised output)
 *   part_lse[slots, rows] fp32 (log2 of each split's softmax denominator)
 * writes out [B, rows, 512] (dtype) and lse [B, rows] fp32 natural log, rows = s_q*heads
 * laid out (s, h).  Sequences with n == 1 are copied through.  Follows mla_decode.py:194-246.
 */
int mla_merge_partials(const float* part_o, const float* part_lse, const int32_t* num_splits,
                       int32_t batch, int32_t rows, int32_t dtype, void* out, float* lse_out,
                       void* stream);

/*
 * The reference's split rule (mla_decode.py:9-30): spread == 0 (even family) or 1
 * (whole-wave family).  Writes the effective split count, blocks per split and
 * number of splits taking one extra block.  Host-only, pure integer.
 */
int mla_split_plan(int32_t seqlen_kv, int32_t num_split, int32_t block_n, int32_t spread,
                   int32_t* ns_out, int32_t* blocks_per_split_out, int32_t* extra_out);

/*
 * The reference's handmade entry point with its exact signature and calling convention
 * (handmade/mla_handmade.py:34-52; its caller binds argtypes [c_void_p] * 7 + [c_int] and
 * restype None, :97-107).  Fixed shape, as the reference's generated kernel: batch 1, 16 query
 * heads, one latent KV head, 8192 cached tokens, fp16, sm_scale = 576^-0.5, contiguous layout
 *   Q [1, 16, 512], Qpe [1, 16, 64], KV [1, 8192, 1, 512], Kpe [1, 8192, 1, 64], out [1, 16, 512].
 * glse (fp16 [1, 16, ns + 64]) and partial (fp16 [1, 16, ns, 576]) are the caller's scratch,
 * as in the reference: glse holds the length and the tile schedule, partial the per-split
 * lse and 16-bit partial rows (the reference's own partial format).  ns = the number of KV
 * splits, 1 .. 128 (forced: the 128 pages cut into ns near-equal ranges).  Runs on the null
 * stream (stream 0) and returns nothing, as the reference; an invalid argument launches
 * nothing and a failure is reported through mla_last_error() (the reference checks nothing).
 */
void mla_launch(const void* Q, const void* Qpe, const void* KV, const void* Kpe, void* glse,
                void* partial, void* out, int ns);

/*
 * Paged KV-cache append: the step before decode that writes the new tokens' latent + rope rows
 * into the paged cache and advances cache_seqlens.  The reference decodes a pre-filled cache
 * and has no append; this is the next row of its path (the cache layout it consumes).  For
 * every sequence b and new token t < n_new:
 *   pos = cache_seqlens[b] + t,  page = block_table[b * block_table_stride + pos / 64],
 *   cache row (page, pos % 64) <- kv_new[b, t, 0..575]   (dims 0..511 latent, 512..575 rope)
 * then cache_seqlens[b] += n_new, in place on the device.  The pages must already be assigned
 * in block_table: if any of a sequence's new positions has pos / 64 >= max_pages or a page id
 * outside [0, num_blocks), none of its rows is written, its length is not advanced and
 * *status (if non-NULL) is set to 1 (the caller clears it).  The cache halves are addressed
 * as in mla_decode_args (one tensor or two views).  Returns 0, MLA_ERR_INVALID (bad shape,
 * pointer, alignment or stride; nothing is launched) or MLA_ERR_HIP.
 */
/*
 * Absorbed value projection after the split-KV pass (the step that consumes the decode's
 * output in an MLA layer; no counterpart in the reference): with the same args as the
 * preceding mla_splitkv_fwd, merge each (sequence, query, head) row's split partials (the
 * combine) and multiply it by that head's up-projection.  For most shapes the merged latent
 * row is formed on chip and never written; when the batch averages 16 or more parts per
 * sequence (num_parts >= 16 * batch, s_q * heads_q <= 16384) the merge runs first as
 * mla_combine_fwd does and writes every multi-split row and its lse into args->out, which the
 * projection then reads.  So args->out is clobbered by this call and cannot hold other data
 * between mla_splitkv_fwd and here (rows of single-split sequences are those the split-KV pass
 * wrote there):
 *   v[b, s, h, n] = sum_k o[b, s, h, k] * W_UV[h][k][n],  k < 512, n < 128,
 * where w_uv_blk holds W_UV k-blocked by 32, w_uv_blk[h][kb][n][kk] = W_UV[h][32 kb + kk][n]
 * ([H, 16, 128, 32] contiguous in the query dtype, 16-byte aligned: each MFMA k-step of 16
 * columns is one contiguous KiB), and v is a contiguous [B, s_q, H, 128] array in that dtype.
 * The merged row is rounded to the query dtype before the product (as mla_combine_fwd would
 * store it); lse is written as by mla_combine_fwd.  Replaces mla_combine_fwd in that
 * pipeline; the output projection by W_O that follows is a plain GEMM.
 */
int mla_combine_absorb(const mla_decode_args* args, const void* w_uv_blk, void* v, void* stream);

typedef struct mla_kv_append_args {
  int32_t batch;   /* B >= 1 */
  int32_t n_new;   /* new tokens per sequence, 1 .. 64 */
  int32_t dtype;   /* MLA_DTYPE_BF16 or MLA_DTYPE_F16 (kv_new and the cache) */
  int32_t num_blocks;
  const void* kv_new;  /* [B, n_new, 576], dims contiguous */
  int64_t new_stride_b, new_stride_t;
  void* kv_nope;       /* cache latent half: page / token strides as in mla_decode_args */
  void* kv_rope;       /* cache rope half */
  int64_t kv_stride_page, kv_stride_tok;
  int64_t kv_rope_stride_page, kv_rope_stride_tok;
  const int32_t* block_table; /* [B, max_pages] */
  int32_t block_table_stride;
  int32_t max_pages;
  int32_t* cache_seqlens;     /* [B], advanced in place */
  int32_t* status;            /* optional device word, set to 1 on a skipped sequence */
  /* MLA_KV_FP8_E4M3: the cache is in the fp8 format of mla_decode_args (kv_nope = e4m3
   * codes, kv_scale = power-of-two scales, kv_rope bf16); kv_new stays bf16 and each new
   * token's latent block j is stored as e4m3(x / 2^k) with 2^k the smallest power of two
   * such that max|x| over the block <= 448 * 2^k (k clamped to [-126, 127]; a zero block
   * gets k = 0), rounded to nearest even. */
  int32_t kv_format;
  int32_t kv_reserved; /* must be 0 */
  float* kv_scale;
  int64_t kv_scale_stride_page, kv_scale_stride_blk;
} mla_kv_append_args;

int mla_kv_append(const mla_kv_append_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLA_DECODE_AMD_H */
