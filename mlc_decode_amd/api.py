"""Paged MLA decode on MI355X: the torch-facing entry points.

* ``get_mla_metadata(cache_seqlens, num_heads_per_head_k, num_heads_k)`` ->
  ``(tile_scheduler_metadata, num_splits)``, the call the reference makes at
  handmade/bench_metax_flashmla.py:31 (schedule algorithm described in
  docs/num_split_design.md:31-135), computed on the GPU by ``mla_get_metadata``.
* ``flash_mla_with_kvcache(q, k_cache, block_table, cache_seqlens, head_dim_v,
  tile_scheduler_metadata, num_splits, softmax_scale=None, causal=False)`` -> ``(out, lse)``,
  the call at handmade/bench_metax_flashmla.py:33-35.
* ``mla_decode_with_kvcache(q, kv_cache, block_table, cache_seqlens, num_splits=None,
  sm_scale=None, causal=True)`` -> ``(out, lse)``: one call that schedules and decodes.
* ``Fp8KVCache`` / ``fp8_kv_cache(num_blocks)`` / ``quantize_kv_cache(kv_cache)``: the fp8
  latent cache (OCP e4m3 codes with power-of-two scales per token and 128 dims, bf16 rope),
  accepted wherever a kv cache is, and written by ``kv_append``.

Tensors live on the GPU; every call goes through the C ABI of ``include/mla_decode_amd.h``
on torch's current stream.  Shapes: q ``[B, s_q, H, 576]``, kv cache ``[num_blocks, 64, 1,
576]`` (or a ``(latent [.., 512], rope [.., 64])`` pair of views), block_table ``[B, P]``
int32, cache_seqlens ``[B]`` int32, out ``[B, s_q, H, 512]`` in q's dtype and lse
``[B, H, s_q]`` fp32 (natural log).
"""
from __future__ import annotations

import ctypes
import os
import math
import threading
from typing import NamedTuple, Optional, Sequence, Tuple, Union

import torch

from . import _lib
from ._lib import (MLA_DIM_QK, MLA_DIM_V, MLA_DTYPE_BF16, MLA_DTYPE_F16, MLA_KV_FP8_E4M3,
                   MLA_KV_NATIVE, MlaDecodeArgs, MlaKvAppendArgs, check)

_DTYPES = {torch.bfloat16: MLA_DTYPE_BF16, torch.float16: MLA_DTYPE_F16}

_ws_lock = threading.Lock()
_workspaces: dict = {}   # (device index, stream handle) -> the buffer calls on that stream use
_retired: list = []      # buffers replaced by larger ones, kept alive until the process ends


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the decode runs only as HIP kernels)")


def workspace(device: torch.device, nbytes: int, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """A cached, 256-byte-aligned device workspace of at least ``nbytes`` bytes for calls
    queued on ``stream`` (torch's current stream of ``device`` by default).

    One buffer per (device, stream), grown on demand, so steady-state calls allocate nothing:
    calls on one stream run in order and can share it, calls on different streams never do.
    A buffer, once handed out, is never freed (a HIP graph captured with its address may
    replay later): when a call needs more, the old buffer is kept alive until the process ends
    and a larger one takes its place.  Sizes grow geometrically (``grown_workspace_size``), so
    the retired buffers of a stream together hold less than its live one.  The returned
    slice's length is the byte count to pass as ``workspace_bytes``.
    """
    nbytes = max(int(nbytes), 256)
    if stream is None:
        stream = torch.cuda.current_stream(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, stream.cuda_stream)
    with _ws_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() - (-buf.data_ptr()) % 256 < nbytes:
            size = grown_workspace_size(None if buf is None else buf.numel(), nbytes + 256)
            if buf is not None:
                _retired.append(buf)
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            _workspaces[key] = buf
    off = (-buf.data_ptr()) % 256
    return buf[off:]


def grown_workspace_size(current: Optional[int], need: int) -> int:
    """Bytes of the buffer that replaces one of ``current`` bytes (None: no buffer yet) when a
    call needs ``need``: the next power of two of at least ``need`` and twice ``current``.  Each
    buffer is then at least twice its predecessor, so the buffers retired on the way to a
    live one sum to less than it, whatever sequence of requests led there."""
    size = 1 << max(int(need) - 1, 1).bit_length()
    if current is not None:
        size = max(size, 2 * int(current))
    return size


def num_parts_for(batch: int, s_q: int, heads_q: int, heads_k: int = 1, cu_count: int = 0) -> int:
    """Schedule parts the decode kernel is laid out for (``mla_num_parts``)."""
    n = _lib.load().mla_num_parts(batch, s_q, heads_q, heads_k, cu_count)
    if n < 1:
        check("mla_num_parts", -n)
    return n


def kernel_variant(rows: int) -> dict:
    """Tile of the main kernel for ``rows`` = s_q * heads query rows (``mla_variant``)."""
    w, t, st, r = (ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32())
    check("mla_variant", _lib.load().mla_variant(rows, ctypes.byref(w), ctypes.byref(t),
                                                  ctypes.byref(st), ctypes.byref(r)))
    kernel = ("mla_wide_kernel" if rows > 32 and os.environ.get("MLA_WIDE", "1") != "0"
              else "mla_splitkv_kernel")
    return {"kernel": kernel, "waves": w.value, "row_tiles_per_wave": t.value, "lds_stages": st.value,
            "rows_per_workgroup": r.value, "stage_tokens": 32}


def get_mla_metadata(cache_seqlens: torch.Tensor, num_heads_per_head_k: int, num_heads_k: int,
                     num_parts: Optional[int] = None, fixed_overhead: int = -1,
                     forced_splits: int = 0, topk: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Tile schedule: ``(tile_scheduler_metadata [num_parts, 8] int32, num_splits [B+1] int32)``.

    ``num_heads_per_head_k`` is ``s_q * h_q // h_kv`` as in the reference's call; it picks
    the kernel's row blocking and hence the part count.  Parts are packed greedily with a
    per-split overhead of ``fixed_overhead`` pages at the reference's payload
    ``ceil(total / parts) + fixed_overhead``; the default (``fixed_overhead < 0``) packs at the
    smallest payload that fits, with the library's overhead ``MLA_DEFAULT_SPLIT_OVERHEAD``.
    ``forced_splits > 0`` cuts every sequence into that many near-equal page ranges instead
    (then ``num_parts = B * forced_splits``).  ``topk`` (sparse decode): every sequence is
    scheduled as ``topk`` keys long, whatever ``cache_seqlens`` holds.
    """
    _require_gpu(cache_seqlens, "cache_seqlens")
    if topk is not None:
        if not 1 <= topk <= _lib.MLA_SPARSE_MAX_TOPK:
            raise ValueError(f"topk must be in [1, {_lib.MLA_SPARSE_MAX_TOPK}]")
        cache_seqlens = torch.full((cache_seqlens.numel(),), topk, dtype=torch.int32, device=cache_seqlens.device)
    if num_heads_k != 1:
        raise ValueError("only one latent KV head (num_heads_k == 1) is supported")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.dim() != 1:
        raise ValueError("cache_seqlens must be a 1-D int32 tensor")
    seqlens = cache_seqlens.contiguous()
    batch = seqlens.numel()
    if forced_splits > 0:
        num_parts = batch * forced_splits
    elif num_parts is None:
        num_parts = num_parts_for(batch, 1, num_heads_per_head_k, 1)
    sched = torch.empty(num_parts, _lib.MLA_SCHED_WORDS, dtype=torch.int32, device=seqlens.device)
    splits = torch.empty(batch + 1, dtype=torch.int32, device=seqlens.device)
    check("mla_get_metadata", _lib.load().mla_get_metadata(
        seqlens.data_ptr(), batch, num_parts, fixed_overhead, forced_splits, sched.data_ptr(),
        splits.data_ptr(), _stream_ptr(seqlens.device)))
    return sched, splits


def get_mla_metadata_host(cache_seqlens: Sequence[int], num_parts: int, fixed_overhead: int = -1,
                          forced_splits: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """The same schedule computed by the library on the host (no GPU needed)."""
    seqlens = torch.as_tensor(list(cache_seqlens), dtype=torch.int32).contiguous()
    batch = seqlens.numel()
    if forced_splits > 0:
        num_parts = batch * forced_splits
    sched = torch.zeros(num_parts, _lib.MLA_SCHED_WORDS, dtype=torch.int32)
    splits = torch.zeros(batch + 1, dtype=torch.int32)
    p32 = lambda t: ctypes.cast(t.data_ptr(), ctypes.POINTER(ctypes.c_int32))  # noqa: E731
    check("mla_get_metadata_host", _lib.load().mla_get_metadata_host(
        p32(seqlens), batch, num_parts, fixed_overhead, forced_splits, p32(sched), p32(splits)))
    return sched, splits


class Fp8KVCache(NamedTuple):
    """The fp8 latent cache: ``latent`` uint8 ``[num_blocks, 64, 512]`` OCP e4m3 codes,
    ``scale`` fp32 ``[num_blocks, 4, 64]`` (power-of-two scale of 128-dim block j of token
    row r at ``[page, j, r]``), ``rope`` bf16 ``[num_blocks, 64, 64]``.  Latent value d of a
    token is ``e4m3(code_d) * scale[d // 128]``.  No counterpart in the reference (its
    design notes list an fp8 KV cache as unexplored, docs/mla_decode_best_implementation.md:1693).
    """
    latent: torch.Tensor
    scale: torch.Tensor
    rope: torch.Tensor


def fp8_kv_cache(num_blocks: int, device="cuda") -> Fp8KVCache:
    """An empty (zero) fp8 cache of ``num_blocks`` pages; fill it with ``kv_append``."""
    return Fp8KVCache(torch.zeros(num_blocks, _lib.MLA_PAGE_TOKENS, MLA_DIM_V, dtype=torch.uint8, device=device),
                      torch.ones(num_blocks, 4, _lib.MLA_PAGE_TOKENS, dtype=torch.float32, device=device),
                      torch.zeros(num_blocks, _lib.MLA_PAGE_TOKENS, MLA_DIM_QK - MLA_DIM_V,
                                  dtype=torch.bfloat16, device=device))


def quantize_kv_cache(kv_cache: torch.Tensor) -> Fp8KVCache:
    """Quantize every page of a bf16 cache ``[num_blocks, 64, 1, 576]`` to the fp8 format
    (on the GPU, through ``mla_kv_append``: page i is appended as one 64-token sequence)."""
    _require_gpu(kv_cache, "kv_cache")
    if kv_cache.dtype != torch.bfloat16 or kv_cache.shape[-1] != MLA_DIM_QK or kv_cache.shape[1] != _lib.MLA_PAGE_TOKENS:
        raise ValueError("kv_cache must be a bf16 [num_blocks, 64, 1, 576] tensor")
    nb = kv_cache.shape[0]
    dst = fp8_kv_cache(nb, kv_cache.device)
    table = torch.arange(nb, dtype=torch.int32, device=kv_cache.device).reshape(nb, 1)
    lens = torch.zeros(nb, dtype=torch.int32, device=kv_cache.device)
    kv_append(kv_cache.reshape(nb, _lib.MLA_PAGE_TOKENS, MLA_DIM_QK), dst, table, lens)
    return dst


def _split_kv(kv_cache) -> Tuple[torch.Tensor, torch.Tensor]:
    if isinstance(kv_cache, Fp8KVCache):
        raise ValueError("an fp8 cache has no bf16 latent half")
    if isinstance(kv_cache, (tuple, list)):
        latent, rope = kv_cache
        if latent.shape[-1] != MLA_DIM_V or rope.shape[-1] != MLA_DIM_QK - MLA_DIM_V:
            raise ValueError("kv pair must be (latent [..., 512], rope [..., 64])")
        return latent, rope
    if kv_cache.shape[-1] != MLA_DIM_QK:
        raise ValueError(f"kv_cache last dim must be {MLA_DIM_QK}")
    return kv_cache[..., :MLA_DIM_V], kv_cache[..., MLA_DIM_V:]


def make_decode_args(q: torch.Tensor, kv_cache, block_table: Optional[torch.Tensor],
                     cache_seqlens: Optional[torch.Tensor], sched: torch.Tensor, splits: torch.Tensor,
                     sm_scale: float, causal: bool, out: Optional[torch.Tensor] = None,
                     lse: Optional[torch.Tensor] = None, indices: Optional[torch.Tensor] = None,
                     status: Optional[torch.Tensor] = None):
    """Validate a paged decode and fill the C ``mla_decode_args`` for it.

    The decode reads no block-table column at or past ``block_table.shape[1]``: a sequence
    whose ``cache_seqlens`` entry exceeds ``64 * block_table.shape[1]`` is decoded over the
    tokens its row covers, and ``status[0]`` (int32, on the device, if given) is set to 1.
    Returns ``(args, out, lse, keep)``; ``keep`` holds the tensors the args point into and
    must stay alive while the args are used.
    """
    _require_gpu(q, "q")
    if q.dim() != 4 or q.shape[-1] != MLA_DIM_QK:
        raise ValueError(f"q must be [B, s_q, H, {MLA_DIM_QK}]")
    if q.dtype not in _DTYPES:
        raise ValueError("q must be bfloat16 or float16")
    fp8 = isinstance(kv_cache, Fp8KVCache)
    if fp8:
        latent, scale, rope = _check_fp8_cache(kv_cache)
        if q.dtype != torch.bfloat16:
            raise ValueError("the fp8 cache is read with bf16 queries")
    else:
        latent, rope = _split_kv(kv_cache)
        scale = None
        for t, n in ((latent, "kv latent"), (rope, "kv rope")):
            _require_gpu(t, n)
            if t.dtype != q.dtype:
                raise ValueError("kv cache dtype must match q")
            if t.dim() != 4 or t.shape[1] != _lib.MLA_PAGE_TOKENS or t.shape[2] != 1 or t.stride(-1) != 1:
                raise ValueError("kv cache must be [num_blocks, 64, 1, D] with unit stride in D")
    B, s_q, H, _ = q.shape
    if indices is not None:  # sparse: keys named by index, no page table or lengths
        _require_gpu(indices, "indices")
        if s_q != 1:
            raise ValueError("the sparse decode takes s_q == 1")
        if indices.dim() == 3:
            if indices.shape[1] != 1:
                raise ValueError("indices must be [B, 1, topk] (s_q == 1)")
            indices = indices[:, 0]
        if indices.dtype != torch.int32 or indices.dim() != 2 or indices.shape[0] != B or indices.stride(1) != 1:
            raise ValueError("indices must be an int32 [B, topk] (or [B, 1, topk]) tensor, unit stride in topk")
        if not 1 <= indices.shape[1] <= _lib.MLA_SPARSE_MAX_TOPK:
            raise ValueError(f"topk must be in [1, {_lib.MLA_SPARSE_MAX_TOPK}]")
        if splits.numel() != B + 1:
            raise ValueError("batch size of q and num_splits disagree")
    else:
        if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
            raise ValueError("block_table must be a [B, P] int32 tensor with unit column stride")
        if cache_seqlens.dtype != torch.int32 or cache_seqlens.dim() != 1:
            raise ValueError("cache_seqlens must be a 1-D int32 tensor")
        if block_table.shape[0] != B or cache_seqlens.shape[0] != B or splits.numel() != B + 1:
            raise ValueError("batch size of q, block_table, cache_seqlens and num_splits disagree")
    if q.stride(-1) != 1:
        raise ValueError("q must have unit stride in its last dim")
    if status is not None:
        _require_gpu(status, "status")
        if status.dtype != torch.int32 or status.numel() < 1:
            raise ValueError("status must be an int32 tensor of at least one element")
    if out is None:
        out = torch.empty(B, s_q, H, MLA_DIM_V, dtype=q.dtype, device=q.device)
    if lse is None:
        lse = torch.empty(B, H, s_q, dtype=torch.float32, device=q.device)
    if lse.shape != (B, H, s_q) or not lse.is_contiguous() or lse.dtype != torch.float32:
        raise ValueError("lse must be a contiguous fp32 [B, H, s_q] tensor")
    if out.shape != (B, s_q, H, MLA_DIM_V) or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must be [B, s_q, H, 512] in q's dtype with unit last stride")
    seqlens = cache_seqlens.contiguous() if cache_seqlens is not None else None
    sched = sched.contiguous()
    splits = splits.contiguous()
    num_parts = sched.shape[0]
    lib = _lib.load()
    ws = workspace(q.device, lib.mla_workspace_bytes(B, s_q, H, num_parts))
    el = q.element_size()
    a = MlaDecodeArgs()
    a.batch, a.s_q, a.heads_q, a.heads_k = B, s_q, H, 1
    a.dtype = _DTYPES[q.dtype]
    a.causal = 1 if causal else 0
    a.sm_scale = float(sm_scale)
    a.num_blocks = latent.shape[0]
    a.q_nope = q.data_ptr()
    a.q_rope = q.data_ptr() + MLA_DIM_V * el
    a.q_stride_b, a.q_stride_s, a.q_stride_h = q.stride(0), q.stride(1), q.stride(2)
    a.q_rope_stride_b, a.q_rope_stride_s, a.q_rope_stride_h = q.stride(0), q.stride(1), q.stride(2)
    a.kv_nope, a.kv_rope = latent.data_ptr(), rope.data_ptr()
    a.kv_stride_page, a.kv_stride_tok, a.kv_stride_batch = latent.stride(0), latent.stride(1), 0
    a.kv_rope_stride_page, a.kv_rope_stride_tok, a.kv_rope_stride_batch = rope.stride(0), rope.stride(1), 0
    a.kv_format = MLA_KV_FP8_E4M3 if fp8 else MLA_KV_NATIVE
    if fp8:
        a.kv_scale = scale.data_ptr()
        a.kv_scale_stride_page, a.kv_scale_stride_blk = scale.stride(0), scale.stride(1)
    if indices is not None:
        a.indices = indices.data_ptr()
        a.indices_stride, a.topk = indices.stride(0), indices.shape[1]
        a.block_table, a.block_table_stride = None, 0
        a.kv_stride_batch = a.kv_rope_stride_batch = 0
    else:
        a.block_table = block_table.data_ptr()
        # one row: its stride is never used, and a view's may be anything
        a.block_table_stride = block_table.stride(0) if B > 1 else block_table.shape[1]
        a.block_table_width = block_table.shape[1]
    a.status = status.data_ptr() if status is not None else None
    a.num_parts = num_parts
    a.cache_seqlens = seqlens.data_ptr() if seqlens is not None else None
    a.tile_sched = sched.data_ptr()
    a.num_splits = splits.data_ptr()
    a.out = out.data_ptr()
    a.o_stride_b, a.o_stride_s, a.o_stride_h = out.stride(0), out.stride(1), out.stride(2)
    a.lse = lse.data_ptr()
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    keep = (q, latent, rope, scale, block_table, seqlens, sched, splits, out, lse, ws, indices, status)
    return a, out, lse, keep


def _decode(q, kv_cache, block_table, cache_seqlens, sched, splits, sm_scale, causal,
            out=None, lse=None, indices=None, status=None, single_split=False):
    """One decode through the C ABI.  ``single_split``: the schedule is known to give every
    sequence one split (forced ``num_splits = 1``), so the split-KV pass finishes every row and
    the combine launch is skipped."""
    a, out, lse, keep = make_decode_args(q, kv_cache, block_table, cache_seqlens, sched, splits,
                                         sm_scale, causal, out, lse, indices, status)
    lib = _lib.load()
    if single_split:
        check("mla_splitkv_fwd", lib.mla_splitkv_fwd(ctypes.byref(a), _stream_ptr(q.device)))
    else:
        check("mla_decode_fwd", lib.mla_decode_fwd(ctypes.byref(a), _stream_ptr(q.device)))
    del keep
    return out, lse


def flash_mla_with_kvcache(q: torch.Tensor, k_cache, block_table: torch.Tensor,
                           cache_seqlens: torch.Tensor, head_dim_v: int,
                           tile_scheduler_metadata: torch.Tensor, num_splits: torch.Tensor,
                           softmax_scale: Optional[float] = None, causal: bool = False,
                           out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                           indices: Optional[torch.Tensor] = None, status: Optional[torch.Tensor] = None):
    """Paged decode with a precomputed schedule -> ``(out [B,s_q,H,512], lse [B,H,s_q])``.

    Same call shape as the reference's use of FlashMLA (handmade/bench_metax_flashmla.py:33-35).
    ``indices`` (int32 ``[B, 1, topk]``, s_q = 1) selects the sparse decode: the keys of sequence
    b are the pool tokens ``indices[b, 0, j]`` (page id * 64 + row; -1 or any id outside the
    cache names no key), ``block_table`` / ``cache_seqlens`` are not read and the schedule must
    come from ``get_mla_metadata(..., topk=topk)``.  No counterpart in the reference's Python
    path: MetaX FlashMLA ships such a kernel (docs/flashmla_metax_analysis.md:43).
    No block-table column at or past ``block_table.shape[1]`` is read: a longer
    ``cache_seqlens`` entry is cut to the table and sets ``status[0] = 1`` (``status``: an
    int32 device tensor the caller clears, optional).
    """
    if head_dim_v != MLA_DIM_V:
        raise ValueError(f"head_dim_v must be {MLA_DIM_V}")
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    return _decode(q, k_cache, block_table, cache_seqlens, tile_scheduler_metadata, num_splits,
                   softmax_scale, causal, out, lse, indices, status)


def prepare_w_uv(w_uv: torch.Tensor) -> torch.Tensor:
    """W_UV ``[H, 512, 128]`` (the per-head latent -> value up-projection) in the layout
    ``mla_combine_absorb`` reads: k-blocked by 32, ``[H, 16, 128, 32]`` contiguous with
    ``blk[h, kb, n, kk] = w_uv[h, 32 * kb + kk, n]``.  Done once per weight."""
    if w_uv.dim() != 3 or w_uv.shape[1] != MLA_DIM_V or w_uv.shape[2] != 128:
        raise ValueError("w_uv must be [H, 512, 128]")
    H = w_uv.shape[0]
    return w_uv.reshape(H, MLA_DIM_V // 32, 32, 128).transpose(2, 3).contiguous()


def mla_decode_absorbed(q: torch.Tensor, kv_cache, block_table: Optional[torch.Tensor],
                        cache_seqlens: Optional[torch.Tensor], tile_scheduler_metadata: torch.Tensor,
                        num_splits: torch.Tensor, w_uv_blk: torch.Tensor, w_o: Optional[torch.Tensor] = None,
                        softmax_scale: Optional[float] = None, causal: bool = False,
                        lse: Optional[torch.Tensor] = None, indices: Optional[torch.Tensor] = None):
    """Decode followed by the absorbed output projection -> ``(y, lse)``.

    The split-KV pass runs as in ``flash_mla_with_kvcache``; its partials are merged straight
    into the per-head product ``v[b, s, h] = o[b, s, h] . W_UV[h]`` (``mla_combine_absorb``,
    ``w_uv_blk`` from ``prepare_w_uv``), so the merged latent output is never written.  ``y`` is
    ``v [B, s_q, H, 128]``, or with ``w_o [H * 128, D]`` the output projection
    ``v.reshape(B, s_q, H * 128) @ w_o`` (a plain GEMM, done by torch).  No counterpart in the
    reference; the step that consumes the decode's ``out [B, s_q, H, 512]`` in DeepSeek MLA.
    """
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    B, s_q, H, _ = q.shape
    if (w_uv_blk.shape != (H, MLA_DIM_V // 32, 128, 32) or w_uv_blk.dtype != q.dtype
            or not w_uv_blk.is_contiguous()):
        raise ValueError("w_uv_blk must be a contiguous [H, 16, 128, 32] tensor in q's dtype (see prepare_w_uv)")
    _require_gpu(w_uv_blk, "w_uv_blk")
    a, out, lse, keep = make_decode_args(q, kv_cache, block_table, cache_seqlens, tile_scheduler_metadata,
                                         num_splits, softmax_scale, causal, None, lse, indices)
    v = torch.empty(B, s_q, H, 128, dtype=q.dtype, device=q.device)
    lib = _lib.load()
    st = _stream_ptr(q.device)
    check("mla_splitkv_fwd", lib.mla_splitkv_fwd(ctypes.byref(a), st))
    check("mla_combine_absorb", lib.mla_combine_absorb(ctypes.byref(a), w_uv_blk.data_ptr(), v.data_ptr(), st))
    del keep
    if w_o is None:
        return v, lse
    if w_o.dim() != 2 or w_o.shape[0] != H * 128 or w_o.dtype != q.dtype:
        raise ValueError("w_o must be [H * 128, D] in q's dtype")
    return torch.matmul(v.reshape(B, s_q, H * 128), w_o), lse


def mla_decode_with_kvcache(q: torch.Tensor, kv_cache, block_table: torch.Tensor,
                            cache_seqlens: torch.Tensor,
                            num_splits: Union[None, int, Tuple[torch.Tensor, torch.Tensor]] = None,
                            sm_scale: Optional[float] = None, causal: bool = True,
                            out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                            status: Optional[torch.Tensor] = None):
    """Schedule + decode in one call -> ``(out, lse)``.

    ``num_splits``: ``None`` = balanced schedule for this GPU; an ``int`` = cut every
    sequence into that many page ranges (1 = the reference's serial baseline: one launch,
    no combine); or a ``(tile_scheduler_metadata, num_splits)`` pair from
    :func:`get_mla_metadata`.  ``status`` as in :func:`flash_mla_with_kvcache`.
    """
    if sm_scale is None:
        sm_scale = MLA_DIM_QK ** -0.5
    if isinstance(num_splits, tuple):
        sched, splits = num_splits
    else:
        forced = int(num_splits) if num_splits is not None else 0
        if num_splits is not None and forced < 1:
            raise ValueError("num_splits must be >= 1")
        sched, splits = get_mla_metadata(cache_seqlens, q.shape[1] * q.shape[2], 1,
                                         forced_splits=forced)
        if forced == 1:
            return _decode(q, kv_cache, block_table, cache_seqlens, sched, splits, sm_scale, causal,
                           out, lse, status=status, single_split=True)
    return _decode(q, kv_cache, block_table, cache_seqlens, sched, splits, sm_scale, causal, out, lse,
                   status=status)


def merge_partials(part_o: torch.Tensor, part_lse: torch.Tensor, num_splits: torch.Tensor,
                   dtype: torch.dtype = torch.bfloat16):
    """LSE-weighted merge of explicit split partials (``mla_merge_partials``).

    part_o ``[slots, rows, 512]`` fp32, part_lse ``[slots, rows]`` fp32 (log2 of each split's
    softmax denominator), num_splits ``[B+1]`` int32 prefix sums -> ``(out [B, rows, 512],
    lse [B, rows])`` with natural-log lse.
    """
    for t, n in ((part_o, "part_o"), (part_lse, "part_lse"), (num_splits, "num_splits")):
        _require_gpu(t, n)
    part_o = part_o.contiguous()
    part_lse = part_lse.contiguous()
    num_splits = num_splits.contiguous()
    batch = num_splits.numel() - 1
    rows = part_o.shape[1]
    out = torch.empty(batch, rows, MLA_DIM_V, dtype=dtype, device=part_o.device)
    lse = torch.empty(batch, rows, dtype=torch.float32, device=part_o.device)
    check("mla_merge_partials", _lib.load().mla_merge_partials(
        part_o.data_ptr(), part_lse.data_ptr(), num_splits.data_ptr(), batch, rows,
        _DTYPES[dtype], out.data_ptr(), lse.data_ptr(), _stream_ptr(part_o.device)))
    return out, lse


def kv_append(kv_new: torch.Tensor, kv_cache, block_table: torch.Tensor,
              cache_seqlens: torch.Tensor, status: Optional[torch.Tensor] = None) -> MlaKvAppendArgs:
    """Append ``kv_new [B, n_new, 576]`` (or ``[B, n_new, 1, 576]``) to the paged cache in
    place and advance ``cache_seqlens`` by ``n_new`` (``mla_kv_append``).

    Token t of sequence b goes to row ``(L_b + t) % 64`` of page
    ``block_table[b, (L_b + t) // 64]``, L_b the length before the call; the pages must already
    be assigned.  A sequence whose new positions run past the table or hit a page id outside
    the cache is left untouched and sets ``status[0] = 1`` when a status tensor (int32, on the
    device) is given.  Nothing is synchronised: the call is queued on the current stream.
    Returns the filled C argument struct (for re-launching through the C ABI directly).
    """
    _require_gpu(kv_new, "kv_new")
    fp8 = isinstance(kv_cache, Fp8KVCache)
    if fp8:
        latent, scale, rope = _check_fp8_cache(kv_cache)
    else:
        latent, rope = _split_kv(kv_cache)
    if kv_new.dim() == 4:
        if kv_new.shape[2] != 1:
            raise ValueError("kv_new [B, n_new, 1, 576] must have one KV head")
        kv_new = kv_new[:, :, 0]
    if kv_new.dim() != 3 or kv_new.shape[-1] != MLA_DIM_QK:
        raise ValueError("kv_new must be [B, n_new, 576]")
    if fp8:
        if kv_new.dtype != torch.bfloat16:
            raise ValueError("the fp8 cache takes bf16 tokens")
    elif kv_new.dtype not in _DTYPES or latent.dtype != kv_new.dtype or rope.dtype != kv_new.dtype:
        raise ValueError("kv_new and the cache must share one 16-bit dtype (bf16 or fp16)")
    B, n_new = kv_new.shape[0], kv_new.shape[1]
    if not fp8 and (latent.dim() != 4 or latent.shape[1] != _lib.MLA_PAGE_TOKENS or latent.shape[2] != 1):
        raise ValueError("kv_cache must be [num_blocks, 64, 1, 576] (or a latent / rope pair)")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != B:
        raise ValueError("block_table must be [B, max_pages] int32")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.shape != (B,) or not cache_seqlens.is_contiguous():
        raise ValueError("cache_seqlens must be a contiguous [B] int32 tensor")
    if kv_new.stride(-1) != 1 or latent.stride(-1) != 1 or rope.stride(-1) != 1:
        raise ValueError("the dims of kv_new and of the cache must be contiguous")
    if status is not None and (status.dtype != torch.int32 or status.numel() < 1):
        raise ValueError("status must be an int32 tensor of at least one element")
    for t, name in ((latent, "kv_cache"), (block_table, "block_table"), (cache_seqlens, "cache_seqlens")):
        _require_gpu(t, name)
    a = MlaKvAppendArgs()
    a.batch, a.n_new, a.dtype, a.num_blocks = B, n_new, _DTYPES[kv_new.dtype], latent.shape[0]
    a.kv_new = kv_new.data_ptr()
    a.new_stride_b, a.new_stride_t = kv_new.stride(0), kv_new.stride(1)
    a.kv_nope, a.kv_rope = latent.data_ptr(), rope.data_ptr()
    a.kv_stride_page, a.kv_stride_tok = latent.stride(0), latent.stride(1)
    a.kv_rope_stride_page, a.kv_rope_stride_tok = rope.stride(0), rope.stride(1)
    a.block_table = block_table.data_ptr()
    a.block_table_stride, a.max_pages = block_table.stride(0), block_table.shape[1]
    a.cache_seqlens = cache_seqlens.data_ptr()
    a.status = status.data_ptr() if status is not None else None
    if fp8:
        a.kv_format = MLA_KV_FP8_E4M3
        a.kv_scale = scale.data_ptr()
        a.kv_scale_stride_page, a.kv_scale_stride_blk = scale.stride(0), scale.stride(1)
    check("mla_kv_append", _lib.load().mla_kv_append(ctypes.byref(a), _stream_ptr(kv_new.device)))
    return a


def _check_fp8_cache(c: Fp8KVCache):
    latent, scale, rope = c.latent, c.scale, c.rope
    for t, n in ((latent, "fp8 latent"), (scale, "fp8 scale"), (rope, "fp8 rope")):
        _require_gpu(t, n)
    nb, page = latent.shape[0], _lib.MLA_PAGE_TOKENS
    if latent.dtype not in (torch.uint8, torch.float8_e4m3fn) or latent.dim() != 3 or \
            latent.shape[1:] != (page, MLA_DIM_V) or latent.stride(-1) != 1:
        raise ValueError("fp8 latent must be a uint8 / float8_e4m3fn [num_blocks, 64, 512] tensor")
    if scale.dtype != torch.float32 or scale.shape != (nb, 4, page) or scale.stride(-1) != 1:
        raise ValueError("fp8 scale must be a float32 [num_blocks, 4, 64] tensor")
    if rope.dtype != torch.bfloat16 or rope.shape != (nb, page, MLA_DIM_QK - MLA_DIM_V) or rope.stride(-1) != 1:
        raise ValueError("fp8 rope must be a bf16 [num_blocks, 64, 64] tensor")
    return latent, scale, rope


def default_sm_scale() -> float:
    return 1.0 / math.sqrt(MLA_DIM_QK)
