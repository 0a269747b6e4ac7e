"""CPU restatement of the reference's MLA decode math -- test infrastructure only.

Functions and the reference code they follow:
  * ``decode_contiguous``  -- test_mla.py:16-27 (``baseline``; same math as
    scripts/check_mla.py:21-32 and baseline_mla.py:167-191): fp32
    ``softmax([q|q_pe].[kv|k_pe]^T * (dim+pe)^-0.5) . kv`` on the contiguous layout.
  * ``decode_paged``       -- the same math on the paged cache, gathered as in
    handmade/bench_metax_flashmla.py:53-61 (``V = K[:, :512]``), generalised to
    per-sequence lengths, causal ``s_q > 1`` (query i sees keys [0, L - s_q + i]) and a
    natural-log LSE ``logsumexp(scale * q.k)`` in the FlashMLA ``[B, H, s_q]`` layout.
  * ``combine``            -- the LSE merge of split partials, mla_decode.py:194-246
    (natural log here, log2 there).
  * ``split_plan``         -- mla_decode.py:9-30.
  * ``schedule_balanced`` / ``schedule_forced`` -- the tile schedule: the greedy packing
    described in docs/num_split_design.md:49-104 and the spread rule of mla_decode.py:9-30.
  * ``append_paged``       -- the paged KV-cache append (no reference counterpart: the
    reference decodes a pre-filled cache; the page/row mapping is the one ``gather``
    reads, handmade/bench_metax_flashmla.py:53-61).
  * ``decode_sparse`` / ``dense_indices`` -- the top-k decode: the same math over the pool
    tokens an index list names (MetaX FlashMLA's sparse kernel, docs/flashmla_metax_analysis.md:43,
    has no source in the reference; pinned by equality with ``decode_paged`` through
    ``dense_indices``, index-permutation invariance and the empty list).
  * ``pack_greedy`` / ``schedule_min_payload`` -- the same greedy loop at an explicit payload
    (no catch-all last part), and the smallest payload in [ceil(total/parts),
    ceil(total/parts) + f] whose packing fits (the library's default schedule).

Pinning (tests/test_oracle.py): ``decode_paged`` against torch's
``scaled_dot_product_attention`` in float64 (a library routine), closed forms (L = 1,
identical keys, q = 0 -> lse = log L), page-permutation and split invariance, s_q = 2
rows against s_q = 1 decodes of L-1 and L, and the committed fixtures in tests/golden/.
``split_plan`` and the schedules are pinned by brute-force coverage / balance checks.
The reference ships no golden vectors for this path.
"""
from __future__ import annotations

import math
from typing import List, Tuple

import torch

PAGE = 64
D_QK = 576
D_V = 512


def decode_contiguous(q, q_pe, kv, k_pe, dtype=torch.float32):
    """q [B,H,512], q_pe [B,H,64], kv [B,L,Hk,512], k_pe [B,L,Hk,64] -> out [B,H,512]."""
    b, h, dim = q.shape
    pe = q_pe.shape[-1]
    hk = kv.shape[2]
    g = h // hk
    query = torch.cat([q, q_pe], -1).to(dtype).reshape(b, hk, g, dim + pe)
    key = torch.cat([kv, k_pe], -1).to(dtype).permute(0, 2, 1, 3)
    scores = torch.matmul(query, key.transpose(-1, -2)) * (dim + pe) ** -0.5
    attn = torch.softmax(scores, -1)
    out = torch.matmul(attn, kv.to(dtype).permute(0, 2, 1, 3))
    return out.reshape(b, h, dim)


def gather(kv_cache: torch.Tensor, table_row: torch.Tensor, L: int) -> torch.Tensor:
    """The first L tokens of one sequence: [L, D] from pages table_row[0..ceil(L/64))."""
    n = (L + PAGE - 1) // PAGE
    pages = kv_cache[table_row[:n].long()]          # [n, 64, D] (or [n, 64, 1, D])
    return pages.reshape(n * PAGE, pages.shape[-1])[:L]


def append_paged(kv_cache: torch.Tensor, block_table: torch.Tensor, cache_seqlens: torch.Tensor,
                 kv_new: torch.Tensor):
    """Write kv_new [B, n, 576] at positions L_b .. L_b+n-1 of each sequence and advance the
    lengths.  A sequence with a position past the table or a page id outside the cache is left
    untouched.  Returns (new cache, new lengths, list of skipped sequences); inputs unchanged."""
    cache = kv_cache.clone()
    lens = cache_seqlens.clone()
    B, n = kv_new.shape[0], kv_new.shape[1]
    P, N = block_table.shape[1], kv_cache.shape[0]
    skipped = []
    for b in range(B):
        L = int(cache_seqlens[b])
        slots = [(L + t) // PAGE for t in range(n)]
        if L < 0 or any(pi >= P for pi in slots) or any(
                not 0 <= int(block_table[b, pi]) < N for pi in slots):
            skipped.append(b)
            continue
        for t in range(n):
            pos = L + t
            cache[int(block_table[b, pos // PAGE]), pos % PAGE, 0, :] = kv_new[b, t]
        lens[b] = L + n
    return cache, lens, skipped


def visible_len(L: int, s_q: int, i: int, causal: bool) -> int:
    return L - (s_q - 1 - i) if causal else L


def decode_paged(q, kv_cache, block_table, cache_seqlens, sm_scale, causal=True, dtype=torch.float32):
    """q [B,s_q,H,576], kv_cache [N,64,1,576] -> (out [B,s_q,H,512], lse [B,H,s_q]).

    Rows with no visible key get out = 0 and lse = -inf.
    """
    B, s_q, H, _ = q.shape
    out = torch.zeros(B, s_q, H, D_V, dtype=dtype)
    lse = torch.full((B, H, s_q), -math.inf, dtype=dtype)
    for b in range(B):
        L = int(cache_seqlens[b])
        if L <= 0:
            continue
        k = gather(kv_cache[:, :, 0, :], block_table[b], L).to(dtype)    # [L, 576]
        v = k[:, :D_V]
        qb = q[b].to(dtype)                                               # [s_q, H, 576]
        scores = torch.matmul(qb, k.t()) * sm_scale                       # [s_q, H, L]
        for i in range(s_q):
            n = visible_len(L, s_q, i, causal)
            if n <= 0:
                continue
            s = scores[i, :, :n]
            lse[b, :, i] = torch.logsumexp(s, -1)
            out[b, i] = torch.matmul(torch.softmax(s, -1), v[:n])
    return out, lse


def decode_sparse(q, kv_cache, indices, sm_scale, dtype=torch.float32):
    """Sparse (top-k) decode: q [B,1,H,576], kv_cache [N,64,1,576], indices [B,1,topk] or
    [B,topk] int -> (out [B,1,H,512], lse [B,H,1]).

    The keys of sequence b are the pool tokens indices[b, j] (page * 64 + row); an index < 0 or
    >= N * 64 names no key.  Rows with no key get out = 0 and lse = -inf.
    """
    B, s_q, H, _ = q.shape
    assert s_q == 1
    idx = indices.reshape(B, -1).to(torch.int64)
    pool = kv_cache.reshape(-1, kv_cache.shape[-1])                        # [N*64, 576]
    out = torch.zeros(B, 1, H, D_V, dtype=dtype)
    lse = torch.full((B, H, 1), -math.inf, dtype=dtype)
    for b in range(B):
        sel = idx[b][(idx[b] >= 0) & (idx[b] < pool.shape[0])]
        if sel.numel() == 0:
            continue
        k = pool[sel].to(dtype)
        s = torch.matmul(q[b, 0].to(dtype), k.t()) * sm_scale              # [H, n]
        lse[b, :, 0] = torch.logsumexp(s, -1)
        out[b, 0] = torch.matmul(torch.softmax(s, -1), k[:, :D_V])
    return out, lse


def dense_indices(block_table, cache_seqlens, topk):
    """The index lists that make decode_sparse equal decode_paged (s_q = 1): token t < L_b of
    sequence b is pool token block_table[b, t // 64] * 64 + t % 64; the rest is -1."""
    B = block_table.shape[0]
    idx = torch.full((B, topk), -1, dtype=torch.int32)
    for b in range(B):
        L = min(int(cache_seqlens[b]), topk)
        t = torch.arange(L)
        idx[b, :L] = (block_table[b, t // PAGE].to(torch.int64) * PAGE + t % PAGE).to(torch.int32)
    return idx


def combine(part_o: torch.Tensor, part_lse: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Merge split partials: part_o [n, ..., 512] (each split softmax-normalised),
    part_lse [n, ...] natural log -> (out [..., 512], lse [...])."""
    lse = torch.logsumexp(part_lse, 0)
    w = torch.exp(part_lse - lse)
    w = torch.nan_to_num(w, nan=0.0)
    return (w.unsqueeze(-1) * part_o).sum(0), lse


def split_plan(seqlen_kv: int, num_split: int, block_n: int, spread: bool = False):
    """(ns, blocks_per_cta, extra) exactly as mla_decode.py:9-30."""
    nb = -(-seqlen_kv // block_n)
    if not spread:
        blocks_per_cta = max(1, -(-(-(-seqlen_kv // num_split)) // block_n))
        ns = max(1, -(-nb // blocks_per_cta))
        return ns, blocks_per_cta, 0
    ns = max(1, min(int(num_split), nb))
    blocks_per_cta, extra = divmod(nb, ns)
    return ns, blocks_per_cta, extra


def pages_of(L: int) -> int:
    return (L + PAGE - 1) // PAGE if L > 0 else 0


def schedule_balanced(seqlens: List[int], num_parts: int, fixed_overhead: int):
    """Greedy packing (docs/num_split_design.md:49-104) -> (records, prefix) where each record
    is (begin_b, begin_page, end_b, end_page, first_split) and prefix is num_splits [B+1]."""
    B = len(seqlens)
    total = sum(pages_of(L) + fixed_overhead for L in seqlens)
    payload = -(-total // num_parts) + fixed_overhead
    now_b = now_p = now_split = cum = 0
    prefix = [0] * (B + 1)
    recs = []
    for p in range(num_parts):
        begin = (now_b, now_p, now_split)
        remain = float("inf") if p == num_parts - 1 else payload
        while now_b < B:
            left = pages_of(seqlens[now_b]) - now_p
            if remain >= left + fixed_overhead:
                cum += now_split + 1
                prefix[now_b + 1] = cum
                remain -= left + fixed_overhead
                now_b, now_p, now_split = now_b + 1, 0, 0
            else:
                take = remain - fixed_overhead
                if take > 0:
                    now_p += int(take)
                    now_split += 1
                break
        recs.append((begin[0], begin[1], now_b, now_p, begin[2]))
    return recs, prefix


def pack_greedy(seqlens: List[int], num_parts: int, payload: int, fixed_overhead: int):
    """The loop of ``schedule_balanced`` with every part, the last included, limited to
    ``payload``.  Returns (records, prefix), or None if the pages do not fit in num_parts
    parts (or the loop stops making progress)."""
    B = len(seqlens)
    f = fixed_overhead
    now_b = now_p = now_split = cum = 0
    prefix = [0] * (B + 1)
    recs = []
    for p in range(num_parts):
        begin = (now_b, now_p, now_split)
        remain = payload
        while now_b < B:
            left = pages_of(seqlens[now_b]) - now_p
            if remain >= left + f:
                cum += now_split + 1
                prefix[now_b + 1] = cum
                remain -= left + f
                now_b, now_p, now_split = now_b + 1, 0, 0
            else:
                take = remain - f
                if take > 0:
                    now_p += take
                    now_split += 1
                break
        recs.append((begin[0], begin[1], now_b, now_p, begin[2]))
    if now_b < B:
        return None
    return recs, prefix


def schedule_min_payload(seqlens: List[int], num_parts: int, fixed_overhead: int):
    """First payload in [lo, lo + f] (lo = ceil(total / parts)) whose greedy packing fits."""
    total = sum(pages_of(L) + fixed_overhead for L in seqlens)
    lo = -(-total // num_parts)
    for payload in range(lo, lo + fixed_overhead + 1):
        got = pack_greedy(seqlens, num_parts, payload, fixed_overhead)
        if got is not None:
            return got[0], got[1], payload
    raise AssertionError("the reference payload always fits")


def schedule_forced(seqlens: List[int], forced: int):
    """Every sequence cut into min(forced, pages) ranges, first ``extra`` one page longer."""
    recs, prefix, cum = [], [0], 0
    for b, L in enumerate(seqlens):
        n = pages_of(L)
        ns = max(1, min(forced, n))
        per, extra = divmod(n, ns)
        for i in range(forced):
            if n == 0:
                recs.append((b, 0, b + 1, 0, 0) if i == 0 else (b + 1, 0, b + 1, 0, 0))
            elif i < ns:
                start = i * per + min(i, extra)
                recs.append((b, start, b, start + per + (1 if i < extra else 0), i))
            else:
                recs.append((b, n, b, n, 0))
        cum += ns
        prefix.append(cum)
    return recs, prefix


def segments(recs, seqlens):
    """Expand records into (part, b, page_begin, page_end, split) segments the way the
    decode kernel walks them."""
    B = len(seqlens)
    out = []
    for p, (bb, bp, eb, ep, fs) in enumerate(recs):
        b, page, split = bb, bp, fs
        while b < B and (b < eb or (b == eb and page < ep)):
            stop = ep if b == eb else pages_of(seqlens[b])
            out.append((p, b, page, stop, split))
            b, page, split = b + 1, 0, 0
    return out
