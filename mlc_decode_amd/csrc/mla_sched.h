// mla_sched.h -- split-KV tile schedule for the MLA decode kernel.
//
// One source, compiled for both the host (mla_get_metadata_host, CPU tests) and the
// device (mla_get_metadata's single-workgroup kernel), so the schedule the GPU uses is
// the schedule the CPU tests check.
//
// The balanced mode follows the algorithm described in the reference's
// docs/num_split_design.md:49-104 (FlashMLA's get_mla_metadata): every part receives
// about total/num_parts 64-token pages plus a fixed per-split overhead, filled greedily
// in (sequence, page) order, cutting a sequence only when the rest of it does not fit.
// The forced mode reproduces the reference's per-sequence split rule (_split_plan,
// spread family, mla_decode.py:9-30) at page granularity.
//
// Part record (MLA_SCHED_WORDS int32 words):
//   [0] begin_b   [1] begin_page   [2] end_b   [3] end_page   [4] split index of the
//   part's first segment   [5..7] zero.
// A part covers positions (b, page) from (begin_b, begin_page) up to, not including,
// (end_b, end_page) in lexicographic order.  A sequence with zero pages is owned by the
// part whose range steps over it (end_b > b), which writes its empty result.
// num_splits[B+1]: prefix sums; sequence b has splits at workspace slots
// num_splits[b] .. num_splits[b+1]-1.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define MLA_HD __host__ __device__
#else
#define MLA_HD
#endif

namespace mla {

constexpr int kPageTokens = 64;
constexpr int kSchedWords = 8;
// Per-split overhead in pages used when the caller passes a negative value: a split
// re-reads the query tile, writes one fp32 partial row block and adds one combine input.
constexpr int kDefaultFixedOverhead = 5;

MLA_HD inline int pages_of(int32_t seqlen) {
  return seqlen > 0 ? (seqlen + kPageTokens - 1) / kPageTokens : 0;
}

MLA_HD inline void sched_write(int32_t* rec, int bb, int bp, int eb, int ep, int split) {
  rec[0] = bb;
  rec[1] = bp;
  rec[2] = eb;
  rec[3] = ep;
  rec[4] = split;
  rec[5] = 0;
  rec[6] = 0;
  rec[7] = 0;
}

// Balanced greedy packing over num_parts parts.  Returns the number of workspace slots.
MLA_HD inline int schedule_balanced(const int32_t* seqlens, int batch, int num_parts,
                                    int fixed_overhead, int32_t* sched, int32_t* num_splits) {
  int64_t total = 0;
  for (int b = 0; b < batch; ++b) total += pages_of(seqlens[b]) + fixed_overhead;
  const int64_t payload = (total + num_parts - 1) / num_parts + fixed_overhead;
  int now_b = 0, now_page = 0, now_split = 0, cum = 0;
  num_splits[0] = 0;
  for (int p = 0; p < num_parts; ++p) {
    const int begin_b = now_b, begin_page = now_page, first_split = now_split;
    // The last part takes whatever is left, so every page is always covered.
    int64_t remain = (p == num_parts - 1) ? (int64_t)1 << 60 : payload;
    while (now_b < batch) {
      const int left = pages_of(seqlens[now_b]) - now_page;
      if (remain >= (int64_t)left + fixed_overhead) {
        cum += now_split + 1;
        num_splits[now_b + 1] = cum;
        remain -= (int64_t)left + fixed_overhead;
        ++now_b;
        now_page = 0;
        now_split = 0;
      } else {
        const int64_t take = remain - fixed_overhead;
        if (take > 0) {
          now_page += (int)take;
          ++now_split;
        }
        break;
      }
    }
    sched_write(sched + p * kSchedWords, begin_b, begin_page, now_b, now_page, first_split);
  }
  return cum;
}

// Every sequence cut into min(forced, pages) near-equal contiguous page ranges; the first
// `extra` ranges take one more page (spread family of the reference's _split_plan).
// num_parts must be batch * forced.  Returns the number of workspace slots.
MLA_HD inline int schedule_forced(const int32_t* seqlens, int batch, int forced, int32_t* sched,
                                  int32_t* num_splits) {
  int cum = 0;
  num_splits[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int np = pages_of(seqlens[b]);
    int ns = forced < np ? forced : np;
    if (ns < 1) ns = 1;
    const int per = np / ns, extra = np % ns;
    for (int i = 0; i < forced; ++i) {
      int32_t* rec = sched + (b * forced + i) * kSchedWords;
      if (np == 0) {
        if (i == 0)
          sched_write(rec, b, 0, b + 1, 0, 0);  // owns the empty sequence
        else
          sched_write(rec, b + 1, 0, b + 1, 0, 0);  // empty part
      } else if (i < ns) {
        const int start = i * per + (i < extra ? i : extra);
        const int len = per + (i < extra ? 1 : 0);
        sched_write(rec, b, start, b, start + len, i);
      } else {
        sched_write(rec, b, np, b, np, 0);  // empty part
      }
    }
    cum += ns;
    num_splits[b + 1] = cum;
  }
  return cum;
}

}  // namespace mla
