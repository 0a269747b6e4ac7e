// mla_sched.h -- split-KV tile schedule for the MLA decode kernel.
//
// One source, compiled for both the host (mla_get_metadata_host, CPU tests) and the
// device (mla_get_metadata's single-workgroup kernel), so the schedule the GPU uses is
// the schedule the CPU tests check.
//
// Packing follows the algorithm described in the reference's docs/num_split_design.md:49-104
// (FlashMLA's get_mla_metadata): parts are filled greedily in (sequence, page) order up to a
// payload, a split costing its pages plus a fixed per-split overhead f, and a sequence is cut
// only when the rest of it does not fit.  Two payloads:
//   balanced     payload = ceil(total / num_parts) + f, the reference's rule;
//   min-payload  the smallest payload in [ceil(total / num_parts), that value] whose packing
//                fits in num_parts parts, i.e. the shortest critical part the greedy rule
//                allows (the library default).
// total = sum over sequences of (pages + f).  The forced mode reproduces the reference's
// per-sequence split rule (_split_plan, spread family, mla_decode.py:9-30) at page granularity.
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

#include "mla_decode_amd.h"

#if defined(__HIPCC__)
#define MLA_HD __host__ __device__
#else
#define MLA_HD
#endif

namespace mla {

constexpr int kPageTokens = 64;
constexpr int kSchedWords = 8;
// Per-split overhead f in pages for the default (min-payload) schedule: a split re-reads the
// query tile, writes one partial row block and adds one combine input.
constexpr int kDefaultSplitOverhead = MLA_DEFAULT_SPLIT_OVERHEAD;
static_assert(kDefaultSplitOverhead >= 0 && kDefaultSplitOverhead < 8, "candidate payload count");

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

// Greedy packing state between sequences: the part being filled, its unused payload and the
// number of splits (workspace slots) so far.
struct PackState {
  int64_t remain;
  int32_t part;
  int32_t cum;
};

// One sequence b of n pages through the greedy packing with payload T and per-split overhead
// f: the inner loop of docs/num_split_design.md:49-104 in closed form (the parts after a cut
// each take T - f pages until the rest fits).  emit(part, b, first_page, split) is called for
// every part that begins inside the sequence, in order.  Returns false if the packing cannot
// place the sequence (T - f < 1 and it does not fit a fresh part).
struct NoEmit {
  MLA_HD void operator()(int, int, int, int) const {}
};
template <class Emit>
MLA_HD inline bool pack_sequence(int b, int n, int64_t T, int f, PackState& st, const Emit& emit) {
  if (st.remain >= (int64_t)n + f) {  // the whole sequence fits the current part
    st.remain -= (int64_t)n + f;
    st.cum += 1;
    return true;
  }
  const int64_t take0 = st.remain - f;  // < n here
  int64_t page = take0 > 0 ? take0 : 0;
  int64_t split = take0 > 0 ? 1 : 0;
  st.part += 1;
  emit(st.part, b, (int)page, (int)split);
  int64_t left = n - page;
  if (T < left + f) {
    const int64_t c = T - f;
    if (c < 1) return false;
    // >= 1 continuation parts of c pages (32-bit division whenever the operands fit, which
    // they do for any real cache: a 64-bit division is a long software sequence on the GPU)
    const int64_t k = (left < (1ll << 31) && c < (1ll << 31))
                          ? (int64_t)(((uint32_t)left + (uint32_t)c - 1u) / (uint32_t)c) - 1
                          : (left + c - 1) / c - 1;
    for (int64_t j = 1; j <= k; ++j) emit(st.part + (int)j, b, (int)(page + j * c), (int)(split + j));
    st.part += (int)k;
    page += k * c;
    split += k;
    left -= k * c;
  }
  st.remain = T - left - f;
  st.cum += (int)split + 1;
  return true;
}

// pack_sequence without the part records, in 32-bit arithmetic and without branches, for
// T + n + f < 2^31 (the device's serial candidate pass, where each step is on the critical
// path): the same rule and the same results.  Both outcomes are computed and one is selected;
// the continuation count k is only computed when the sequence is cut and its rest does not fit
// a fresh part (then c = T - f >= 1 is required, as in pack_sequence).
MLA_HD inline bool pack_sequence32(int n, int T, int f, int& remain, int& part, int& cum) {
  const bool fits = remain >= n + f;
  const int take0 = remain - f;
  const int page = take0 > 0 ? take0 : 0;
  const int split0 = take0 > 0 ? 1 : 0;
  int left = n - page;  // > 0 whenever the sequence does not fit
  const bool cut = !fits && T < left + f;
  const int c = T - f;
  const uint32_t cu = c > 0 ? (uint32_t)c : 1u;
  const int k = cut ? (int)(((uint32_t)left + cu - 1u) / cu) - 1 : 0;
  left -= k * c;
  const bool ok = !cut || c >= 1;
  remain = fits ? remain - (n + f) : T - left - f;
  part += fits ? 0 : 1 + k;
  cum += fits ? 1 : split0 + k + 1;
  return ok;
}

// Sum over sequences of pages + f, and the payload bounds [lo, hi]: no packing fits num_parts
// parts below lo, and the greedy packing always fits at hi (every closed part consumes at
// least hi - f of the total).
MLA_HD inline void payload_bounds(int64_t total, int num_parts, int f, int64_t* lo, int64_t* hi) {
  *lo = (total + num_parts - 1) / num_parts;
  *hi = *lo + f;
}

// Does the greedy packing with payload T fit in num_parts parts?
MLA_HD inline bool packing_fits(const int32_t* pages, int batch, int num_parts, int64_t T, int f) {
  PackState st{T, 0, 0};
  for (int b = 0; b < batch; ++b)
    if (!pack_sequence(b, pages[b], T, f, st, NoEmit{}) || st.part >= num_parts) return false;
  return true;
}

// Writes the records and num_splits of the greedy packing with payload T (which must fit).
// Parts after the last used one are empty records at (batch, 0).  Returns the slot count.
MLA_HD inline int write_packing(const int32_t* pages, int batch, int num_parts, int64_t T, int f,
                                int32_t* sched, int32_t* num_splits) {
  sched_write(sched, 0, 0, batch, 0, 0);
  const auto emit = [&](int p, int b, int page, int split) {
    if (p < num_parts) sched_write(sched + p * kSchedWords, b, page, batch, 0, split);
    if (p - 1 < num_parts) {
      sched[(p - 1) * kSchedWords + 2] = b;
      sched[(p - 1) * kSchedWords + 3] = page;
    }
  };
  PackState st{T, 0, 0};
  num_splits[0] = 0;
  for (int b = 0; b < batch; ++b) {
    pack_sequence(b, pages[b], T, f, st, emit);
    num_splits[b + 1] = st.cum;
  }
  for (int p = st.part + 1; p < num_parts; ++p) sched_write(sched + p * kSchedWords, batch, 0, batch, 0, 0);
  return st.cum;
}

// Host driver of both payload rules (pages computed into a scratch array of batch entries).
// min_payload = false: the reference's payload; true: the smallest payload that fits.
inline int schedule_packed(const int32_t* seqlens, int batch, int num_parts, int f,
                           bool min_payload, int32_t* pages, int32_t* sched,
                           int32_t* num_splits) {
  int64_t total = 0;
  for (int b = 0; b < batch; ++b) {
    pages[b] = pages_of(seqlens[b]);
    total += pages[b] + f;
  }
  int64_t lo, hi;
  payload_bounds(total, num_parts, f, &lo, &hi);
  int64_t T = hi;
  if (min_payload)
    for (int64_t c = lo; c < hi; ++c)
      if (packing_fits(pages, batch, num_parts, c, f)) {
        T = c;
        break;
      }
  return write_packing(pages, batch, num_parts, T, f, sched, num_splits);
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
