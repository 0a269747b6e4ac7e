"""Drop-in ``mla_decode`` for MI355X: the reference module's names over one HIP kernel.

Every factory returns an :class:`mlc_decode_amd.MlaKernel`, called as
``kernel(q, q_pe, kv, k_pe, output)`` (reference mla_decode.py:66-72).  The TileLang-only
knobs of the reference (block_N, block_H, num_stages, dim_chunk_num, threads,
combine_groups, combine_threads, q_in_reg) are validated and recorded but do not change the
kernel: tiles, stages and waves are fixed per head count by the HIP library, KV pages are
64 tokens, and only ``num_split`` / ``spread`` (how many page ranges each sequence is cut
into) carry over.
"""
from __future__ import annotations

import ctypes
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from mlc_decode_amd import _lib  # noqa: E402
from mlc_decode_amd._lib import check  # noqa: E402
from mlc_decode_amd.legacy import MlaKernel  # noqa: E402

PAGE_TOKENS = 64
_TUNE_SPLITS = (1, 2, 4, 8, 16, 32, 64)   # forced per-sequence split counts tried by autotune
_TUNE_MAX_NUM_SPLIT = 1024


def _split_plan(seqlen_kv, num_split, block_n, spread=False):
    """``(ns, blocks_per_cta, extra)`` for cutting ceil(seqlen_kv/block_n) blocks into
    ``num_split`` CTAs -- the reference rule of mla_decode.py:9-30, computed by the library
    (``mla_split_plan``)."""
    ns, bpc, extra = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    check("mla_split_plan", _lib.load().mla_split_plan(
        int(seqlen_kv), int(num_split), int(block_n), 1 if spread else 0,
        ctypes.byref(ns), ctypes.byref(bpc), ctypes.byref(extra)))
    return ns.value, bpc.value, extra.value


def _check_knobs(block_N=64, block_H=16, num_stages=1, dim_chunk_num=8, threads=128,
                 combine_groups=1, combine_threads=64):
    if block_N not in (16, 32, 64):
        raise ValueError("block_N must be 16, 32 or 64 (KV is consumed in 64-token pages)")
    if block_H < 1 or num_stages < 0 or dim_chunk_num < 1 or threads < 64 or threads % 64:
        raise ValueError("invalid block_H / num_stages / dim_chunk_num / threads")
    if combine_groups < 1 or combine_threads < 1:
        raise ValueError("invalid combine_groups / combine_threads")


def _make(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, num_split, spread, softmax_scale, cfg):
    # Splits are cut at 64-token page granularity on MI355X.
    ns = _split_plan(seqlen_kv, max(1, int(num_split)), PAGE_TOKENS, spread)[0]
    return MlaKernel(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, splits=ns, config=cfg,
                     sm_scale=softmax_scale)


def flashattn_shared_q(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, block_N, block_H,
                       num_split, num_stages, dim_chunk_num, softmax_scale, threads=128,
                       spread=False, combine_groups=1, combine_threads=64):
    """Explicit-config kernel (reference mla_decode.py:36-39)."""
    _check_knobs(block_N, block_H, num_stages, dim_chunk_num, threads, combine_groups, combine_threads)
    cfg = dict(block_N=block_N, block_H=block_H, num_split=num_split, num_stages=num_stages,
               dim_chunk_num=dim_chunk_num, threads=threads, spread=spread,
               combine_groups=combine_groups, combine_threads=combine_threads, q_in_reg=False)
    return _make(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, num_split, spread,
                 softmax_scale, cfg)


def flashattn_frag_q(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, block_N, block_H,
                     num_split, num_stages, dim_chunk_num, softmax_scale, threads=128,
                     spread=False, combine_groups=1, combine_threads=64):
    """Same kernel: on MI355X the query tile always lives in registers."""
    k = flashattn_shared_q(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, block_N, block_H,
                           num_split, num_stages, dim_chunk_num, softmax_scale, threads, spread,
                           combine_groups, combine_threads)
    k.config["q_in_reg"] = True
    return k


def mla_autotune_configs(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim):
    """Candidate configs (reference mla_decode.py:539-606 format).  ``num_split=None`` is
    the balanced schedule for this GPU; the others force that many splits per sequence."""
    pages = -(-seqlen_kv // PAGE_TOKENS)
    block_h = min(16, heads // kv_head_num)
    base = dict(block_N=PAGE_TOKENS, block_H=block_h, num_stages=1, dim_chunk_num=8,
                q_in_reg=True, threads=64 * 4, combine_groups=1)
    out = [dict(base, num_split=None, spread=True)]
    for ns in _TUNE_SPLITS:
        if ns <= pages and ns <= _TUNE_MAX_NUM_SPLIT:
            out.append(dict(base, num_split=ns, spread=True))
    return out


def build_kernel_from_config(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, cfg):
    """Kernel for an explicit config (reference mla_decode.py:720-729)."""
    ns = cfg.get("num_split")
    softmax_scale = (dim + pe_dim) ** -0.5
    if ns is None:
        return MlaKernel(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, splits=None,
                         config=cfg, sm_scale=softmax_scale)
    _check_knobs(cfg.get("block_N", PAGE_TOKENS), cfg.get("block_H", 16), cfg.get("num_stages", 1),
                 cfg.get("dim_chunk_num", 8), cfg.get("threads", 128), cfg.get("combine_groups", 1),
                 cfg.get("combine_threads", 64))
    return _make(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, ns, cfg.get("spread", False),
                 softmax_scale, dict(cfg))


def _bench(kernel, args, warmup=5, rep=20):
    import torch
    out = torch.empty_like(args[0])
    for _ in range(warmup):
        kernel(*args, out)
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(rep):
        kernel(*args, out)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / rep * 1000.0


def flashattn_autotuned(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, **cfg):
    """Times every candidate of :func:`mla_autotune_configs` on random inputs and returns
    the fastest kernel (reference mla_decode.py:609-620); explicit knobs skip the search."""
    if cfg:
        return build_kernel_from_config(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, cfg)
    import torch
    dev = torch.device("cuda")
    g = torch.Generator(device="cpu").manual_seed(0)
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.1).to(torch.float16).to(dev)  # noqa: E731
    args = (mk(batch, heads, dim), mk(batch, heads, pe_dim), mk(batch, seqlen_kv, kv_head_num, dim),
            mk(batch, seqlen_kv, kv_head_num, pe_dim))
    best = None
    for c in mla_autotune_configs(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim):
        k = build_kernel_from_config(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, c)
        us = _bench(k, args)
        if best is None or us < best[0]:
            best = (us, k)
    best[1].config["latency_us"] = round(best[0], 3)
    return best[1]


_CACHE_SHARED = {}
_CACHE_FRAG = {}
_TUNE_CACHE = {}
_AUTOTUNE_ENABLED = os.environ.get("MLA_NO_AUTOTUNE", "0") != "1"


def _legacy_kernel(batch, heads, kv_heads, kv_ctx, dim, pe_dim):
    """No-search path: the balanced schedule for this GPU."""
    key = (batch, heads, kv_heads, kv_ctx, dim, pe_dim)
    k = _CACHE_SHARED.get(key)
    if k is None:
        k = MlaKernel(batch, heads, kv_heads, kv_ctx, dim, pe_dim, splits=None)
        _CACHE_SHARED[key] = k
    return k


def _get_kernel(batch, heads, kv_heads, kv_ctx, dim, pe_dim):
    """Kernel for a shape (reference mla_decode.py:690-710): autotuned once per shape unless
    MLA_NO_AUTOTUNE=1; a failed search falls back to the balanced schedule."""
    key = (batch, heads, kv_heads, kv_ctx, dim, pe_dim)
    if _AUTOTUNE_ENABLED:
        k = _TUNE_CACHE.get(key)
        if k is not None:
            return k
        try:
            k = flashattn_autotuned(batch, heads, kv_heads, kv_ctx, dim, pe_dim)
        except (RuntimeError, ValueError) as exc:
            print(f"[mla_decode] autotune failed ({type(exc).__name__}: {exc}); "
                  f"using the balanced schedule", file=sys.stderr)
        else:
            _TUNE_CACHE[key] = k
            return k
    return _legacy_kernel(batch, heads, kv_heads, kv_ctx, dim, pe_dim)


def run_kernel(q, q_pe, kv, k_pe, output, batch, heads, kv_heads, kv_ctx, dim, pe_dim):
    kernel = _get_kernel(int(batch), int(heads), int(kv_heads), int(kv_ctx), int(dim), int(pe_dim))
    kernel(q, q_pe, kv, k_pe, output)
