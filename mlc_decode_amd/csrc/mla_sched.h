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

// pack_sequence with the part records, in 32-bit arithmetic, for payloads T >= f + 1 with
// T + n + f < 2^31 (the device's parallel schedule): the same rule and the same records.
template <class Emit>
MLA_HD inline void pack_sequence_emit32(int b, int n, int T, int f, int& remain, int& part, int& cum,
                                        const Emit& emit) {
  if (remain >= n + f) {
    remain -= n + f;
    cum += 1;
    return;
  }
  const int take0 = remain - f;
  const int page = take0 > 0 ? take0 : 0;
  const int split0 = take0 > 0 ? 1 : 0;
  part += 1;
  emit(part, b, page, split0);
  int left = n - page;
  int k = 0;
  if (T < left + f) {
    const uint32_t c = (uint32_t)(T - f);
    k = (int)(((uint32_t)left + c - 1u) / c) - 1;
    for (int j = 1; j <= k; ++j) emit(part + j, b, page + j * (int)c, split0 + j);
    part += k;
    left -= k * (int)c;
  }
  remain = T - left - f;
  cum += split0 + k + 1;
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
MLA_HD inline int forced_count(int np, int forced) {
  const int ns = forced < np ? forced : np;
  return ns < 1 ? 1 : ns;
}
// Record i of sequence b (np pages), at sched + (b * forced + i) * kSchedWords.
MLA_HD inline void forced_record(int b, int i, int np, int forced, int32_t* sched) {
  const int ns = forced_count(np, forced);
  const int per = np / ns, extra = np % ns;
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
MLA_HD inline int schedule_forced(const int32_t* seqlens, int batch, int forced, int32_t* sched,
                                  int32_t* num_splits) {
  int cum = 0;
  num_splits[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int np = pages_of(seqlens[b]);
    for (int i = 0; i < forced; ++i) forced_record(b, i, np, forced, sched);
    cum += forced_count(np, forced);
    num_splits[b + 1] = cum;
  }
  return cum;
}

// ---------------------------------------------------------------------------------------
// Closed form of the greedy packing between resets (the device's parallel schedule).
//
// Call a sequence a *reset* when it does not fit the current part and at most f pages of
// payload are left there (remain <= f and remain < n + f): it leaves that remain unused and
// starts at page 0 of a fresh part, as the first sequence does.  Let S_i be the exclusive
// prefix sum of (pages + f) and A = S_i - S_r the cost accumulated since the last reset r
// (r = 0 for the first sequence, S_0 = 0).  With c = T - f >= 1, the state entering each
// sequence i > r, up to and including the next reset, is
//   remain = T - A                         if A <= T (still inside the part the reset opened)
//          = c - 1 - ((A - f - 1) mod c)    otherwise
//   part   = p_r + (A > T ? floor((A - f - 1) / c) : 0)
//   cum    = part + i - (number of resets at indices 1 .. i-1)
// where p_r is the part reset r opened (0 for r = 0, else the part entering r plus one).
// Proof by induction on i: a step that fits maps remain x to x - n - f; a cut with remain > f
// leaves ((n - (x - f) - 1) mod c) + 1 pages in its last part, so x' = c - 1 - ((n + f - 1 - x)
// mod c) and the part index grows by ceil((n - x + f) / c); both agree with A' = A + n + f.
// (A sequence with n >= 1 that fits also satisfies the mod form, since x' <= c - 1.)  So the
// serial pass reduces to finding each next reset, which one wave does for 64 sequences at a
// time; everything else is per-sequence arithmetic on the prefix sums.  Needs every quantity
// below 2^31 (the device uses it while the total is below 2^30) and c >= 1: with c < 1 no
// sequence with pages can be placed, so such a payload fails unless every sequence is empty.
// ---------------------------------------------------------------------------------------
constexpr int kWalkWin = 64;  // sequences per walk window (one wave)

MLA_HD inline int walk_remain(int A, int T, int f, int c) {
  return A <= T ? T - A : c - 1 - (int)((uint32_t)(A - f - 1) % (uint32_t)c);
}
MLA_HD inline int walk_parts(int A, int T, int f, int c) {
  return A > T ? (int)((uint32_t)(A - f - 1) / (uint32_t)c) : 0;
}
MLA_HD inline bool walk_is_reset(int remain, int n, int f) { return remain <= f && remain < n + f; }

// walk_remain from residues, without a division: e = A mod c, formed as (S_k mod c - S_r mod c)
// mod c, and f1 = (f + 1) mod c; then (A - f - 1) mod c = (e - f1) mod c.  A > T implies
// A - f - 1 > 0, so this is the same value as walk_remain's.
MLA_HD inline int mod_sub(int a, int b, int c) {  // (a - b) mod c for a, b in [0, c)
  const int e = a - b;
  return e < 0 ? e + c : e;
}
MLA_HD inline int walk_remain_res(int A, int e, int T, int f1, int c) {
  return A <= T ? T - A : c - 1 - mod_sub(e, f1, c);
}

// Lookahead of sequence i: the first d in 1 .. kWalkLook with i + d < batch that is a reset if
// i is one (0 if none), and the part increment at it.  The walk follows these links from
// reset to reset and searches further only where a link is missing.  sig(k) = S[k] mod c.
constexpr int kWalkLook = 8;
template <class Sig>
MLA_HD inline int walk_lookahead(const int32_t* S, int i, int batch, int T, int f, int c, int f1, const Sig& sig,
                                 int* inc) {
  const int Si = S[i], si = sig(i);
  for (int d = 1; d <= kWalkLook && i + d < batch; ++d) {
    const int k = i + d;
    const int A = S[k] - Si;
    if (walk_is_reset(walk_remain_res(A, mod_sub(sig(k), si, c), T, f1, c), S[k + 1] - S[k] - f, f)) {
      *inc = walk_parts(A, T, f, c) + 1;
      return d;
    }
  }
  *inc = 0;
  return 0;
}

// Walk state at a window start: S of the last reset, the part it opened, resets so far.
struct WalkEntry {
  int32_t rs, p, w;
};

// The state entering sequence m, from the entry of its window and the window's reset mask
// restricted to lanes below m's (S: the prefix sums, batch + 1 entries).
MLA_HD inline PackState walk_state(const int32_t* S, int m, WalkEntry e, uint64_t before, int T, int f,
                                   int c) {
  const int base = m - (m % kWalkWin);
  while (before != 0) {
    const int j = __builtin_ctzll(before);  // resets in lane order
    before &= before - 1;
    const int Sj = S[base + j];
    e.p += walk_parts(Sj - e.rs, T, f, c) + 1;
    e.w += 1;
    e.rs = Sj;
  }
  const int A = S[m] - e.rs;
  const int part = e.p + walk_parts(A, T, f, c);
  return PackState{walk_remain(A, T, f, c), part, part + m - e.w};
}

#if !defined(__HIP_DEVICE_COMPILE__)
// Host emulation of the device's walk for one payload T: the same windows, entries, masks and
// lookahead links (lane loops where the device uses a ballot).  ent/msk: one entry per
// window.  Returns the final part index, or -1 if T cannot place a sequence (c < 1).
inline int walk_payload_host(const int32_t* S, int batch, int T, int f, WalkEntry* ent, uint64_t* msk) {
  const int c = T - f;
  if (c < 1) return -1;
  const int f1 = (f + 1) % c;
  const auto sig = [&](int k) { return S[k] % c; };
  int rs = 0, rsig = 0, p = 0, w = 0;
  int pend = -1, pend_inc = 0;  // a reset in the next window, reached by a link
  const int nwin = (batch + kWalkWin - 1) / kWalkWin;
  for (int win = 0; win < nwin; ++win) {
    const int base = win * kWalkWin;
    ent[win] = WalkEntry{rs, p, w};
    uint64_t mask = 0;
    int cur = -1;  // lane of the last reset in this window
    const auto take = [&](int lane, int inc) {
      p += inc;
      w += 1;
      rs = S[base + lane];
      rsig = sig(base + lane);
      mask |= 1ull << lane;
      cur = lane;
    };
    if (pend >= 0) take(pend, pend_inc), pend = -1;
    for (;;) {
      int from = 0;  // first lane the search may find
      if (cur >= 0) {
        int inc, d = walk_lookahead(S, base + cur, batch, T, f, c, f1, sig, &inc);
        while (d > 0 && cur + d < kWalkWin) {
          take(cur + d, inc);
          d = walk_lookahead(S, base + cur, batch, T, f, c, f1, sig, &inc);
        }
        if (d > 0) {
          pend = cur + d - kWalkWin;
          pend_inc = inc;
          break;
        }
        from = cur + kWalkLook + 1;
      }
      int found = -1;
      for (int lane = from; lane < kWalkWin && base + lane < batch; ++lane) {
        const int i = base + lane;
        const int A = S[i] - rs;
        if (i > 0 && walk_is_reset(walk_remain_res(A, mod_sub(sig(i), rsig, c), T, f1, c), S[i + 1] - S[i] - f, f)) {
          found = lane;
          break;
        }
      }
      if (found < 0) break;
      take(found, walk_parts(S[base + found] - rs, T, f, c) + 1);
    }
    msk[win] = mask;
  }
  return p + walk_parts(S[batch] - rs, T, f, c);
}

// The whole schedule through the walk, as the device builds it: prefix sums, one walk per
// candidate payload, then every sequence's records from its own entry state.  Returns the
// slot count, or -1 where the device falls back to the serial pass (total >= 2^30 or no
// sequence has pages).  S: batch + 1 entries; ent, msk: kMetaCand * windows entries.
inline int schedule_walk_host(const int32_t* seqlens, int batch, int num_parts, int f, bool min_payload,
                              int32_t* S, WalkEntry* ent, uint64_t* msk, int32_t* sched,
                              int32_t* num_splits) {
  int64_t total = 0;
  int maxn = 0;
  for (int b = 0; b < batch; ++b) {
    const int n = pages_of(seqlens[b]);
    maxn = n > maxn ? n : maxn;
    S[b] = (int32_t)total;
    total += n + f;
    if (total >= (1ll << 30)) return -1;
  }
  S[batch] = (int32_t)total;
  if (maxn == 0) return -1;
  int64_t lo, hi;
  payload_bounds(total, num_parts, f, &lo, &hi);
  const int ncand = min_payload ? (int)(hi - lo) + 1 : 1;
  const int nwin = (batch + kWalkWin - 1) / kWalkWin;
  int best = ncand - 1, last = -1;
  for (int ci = ncand - 1; ci >= 0; --ci) {
    const int T = (int)(min_payload ? lo + ci : hi);
    const int fin = walk_payload_host(S, batch, T, f, ent + ci * nwin, msk + ci * nwin);
    if (fin >= 0 && fin < num_parts) best = ci, last = fin;
  }
  const int T = (int)(min_payload ? lo + best : hi), c = T - f;
  sched_write(sched, 0, 0, batch, 0, 0);
  num_splits[0] = 0;
  const auto emit = [&](int p, int b, int page, int split) {
    if (p < num_parts) sched_write(sched + p * kSchedWords, b, page, batch, 0, split);
    if (p - 1 < num_parts) {
      sched[(p - 1) * kSchedWords + 2] = b;
      sched[(p - 1) * kSchedWords + 3] = page;
    }
  };
  for (int m = 0; m < batch; ++m) {
    const int win = m / kWalkWin, lane = m % kWalkWin;
    const PackState st = walk_state(S, m, ent[best * nwin + win],
                                    msk[best * nwin + win] & ((1ull << lane) - 1), T, f, c);
    int remain = (int)st.remain, part = st.part, cum = st.cum;
    pack_sequence_emit32(m, S[m + 1] - S[m] - f, T, f, remain, part, cum, emit);
    num_splits[m + 1] = cum;
  }
  for (int p = last + 1; p < num_parts; ++p) sched_write(sched + p * kSchedWords, batch, 0, batch, 0, 0);
  return num_splits[batch];
}
#endif

}  // namespace mla
