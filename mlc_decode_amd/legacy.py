"""Kernel objects for the reference's contiguous-cache call shape.

The reference's kernels are called as ``kernel(q, q_pe, kv, k_pe, output)`` with
``q [B, H, 512]``, ``q_pe [B, H, 64]``, ``kv [B, L, 1, 512]``, ``k_pe [B, L, 1, 64]``,
``output [B, H, 512]`` (mla_decode.py:66-72, test_mla.py:30-58).  ``MlaKernel`` runs that
call on the same split-KV HIP kernel as the paged path (the C ABI's contiguous mode:
no block table, per-batch strides), with its split policy fixed at construction:
  * ``splits=None``: the balanced schedule for this GPU (mla_decode._get_kernel);
  * ``splits=n``: every sequence cut into n page ranges (n = 1 is the serial baseline of
    baseline_mla._get_kernel; explicit configs of build_kernel_from_config).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from ._lib import MLA_DIM_V, MlaDecodeArgs, check
from .api import _DTYPES, _stream_ptr, get_mla_metadata, workspace

DIM = 512
PE_DIM = 64


class MlaKernel:
    """``kernel(q, q_pe, kv, k_pe, output=None)`` for fixed (batch, heads, kv_ctx)."""

    def __init__(self, batch: int, heads: int, kv_heads: int, kv_ctx: int, dim: int = DIM,
                 pe_dim: int = PE_DIM, splits: Optional[int] = None, config: Optional[dict] = None,
                 sm_scale: Optional[float] = None):
        if kv_heads != 1:
            raise ValueError("only kv_heads == 1 (one shared latent head) is supported")
        if dim != DIM or pe_dim != PE_DIM:
            raise ValueError(f"MLA decode is built for dim={DIM}, pe_dim={PE_DIM}")
        if batch < 1 or heads < 1 or kv_ctx < 1:
            raise ValueError("batch, heads and kv_ctx must be >= 1")
        if splits is not None and splits < 1:
            raise ValueError("splits must be >= 1")
        self.batch, self.heads, self.kv_heads, self.kv_ctx = batch, heads, kv_heads, kv_ctx
        self.dim, self.pe_dim = dim, pe_dim
        self.splits = splits
        self.config = dict(config or {})
        self.sm_scale = float(sm_scale) if sm_scale is not None else (dim + pe_dim) ** -0.5
        if not self.sm_scale > 0:
            raise ValueError("sm_scale must be > 0")
        self._state = {}  # device -> (seqlens, sched, num_splits)
        self._prepared = None  # (key of the last call's tensors, its prepared C arguments)

    def __repr__(self) -> str:
        pol = "balanced" if self.splits is None else f"{self.splits} split(s)/sequence"
        return (f"MlaKernel(batch={self.batch}, heads={self.heads}, kv_ctx={self.kv_ctx}, "
                f"{pol})")

    def _schedule(self, device: torch.device):
        key = (device.type, device.index)
        st = self._state.get(key)
        if st is None:
            seqlens = torch.full((self.batch,), self.kv_ctx, dtype=torch.int32, device=device)
            sched, nsplits = get_mla_metadata(seqlens, self.heads, 1,
                                              forced_splits=self.splits or 0)
            st = (seqlens, sched, nsplits)
            self._state[key] = st
        return st

    @staticmethod
    def _key(q, q_pe, kv, k_pe, output):
        """Everything the prepared arguments depend on: pointers, shapes, strides, dtypes,
        the device and torch's current stream on it."""
        ts = (q, q_pe, kv, k_pe)
        return (tuple((t.data_ptr(), t.shape, t.stride(), t.dtype, t.device) for t in ts),
                None if output is None else (output.data_ptr(), output.shape, output.stride(), output.dtype),
                torch.cuda.current_stream(q.device).cuda_stream if q.is_cuda else None)

    def _prepare(self, q, q_pe, kv, k_pe, output):
        """Validate one call's tensors and fill the C arguments for them (output fields aside)."""
        B, H, L = self.batch, self.heads, self.kv_ctx
        for t, name, shape in ((q, "q", (B, H, DIM)), (q_pe, "q_pe", (B, H, PE_DIM)),
                               (kv, "kv", (B, L, 1, DIM)), (k_pe, "k_pe", (B, L, 1, PE_DIM))):
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {shape}")
            if not t.is_cuda:
                raise ValueError(f"{name} must be a GPU tensor")
            if t.dtype != q.dtype:
                raise ValueError("q, q_pe, kv and k_pe must share one dtype")
            if t.stride(-1) != 1:
                raise ValueError(f"{name} must have unit stride in its last dim")
        if q.dtype not in _DTYPES:
            raise ValueError("dtype must be float16 or bfloat16")
        if output is not None and (tuple(output.shape) != (B, H, DIM) or output.dtype != q.dtype
                                   or output.stride(-1) != 1):
            raise ValueError("output must be [B, H, 512] in the input dtype")
        seqlens, sched, nsplits = self._schedule(q.device)
        lib = _lib.load()
        num_parts = sched.shape[0]
        ws = workspace(q.device, lib.mla_workspace_bytes(B, 1, H, num_parts))
        a = MlaDecodeArgs()
        a.batch, a.s_q, a.heads_q, a.heads_k = B, 1, H, 1
        a.dtype = _DTYPES[q.dtype]
        a.causal = 0
        a.sm_scale = float(self.sm_scale)
        a.num_blocks = 1
        a.q_nope, a.q_rope = q.data_ptr(), q_pe.data_ptr()
        a.q_stride_b, a.q_stride_s, a.q_stride_h = q.stride(0), 0, q.stride(1)
        a.q_rope_stride_b, a.q_rope_stride_s, a.q_rope_stride_h = q_pe.stride(0), 0, q_pe.stride(1)
        a.kv_nope, a.kv_rope = kv.data_ptr(), k_pe.data_ptr()
        a.kv_stride_page, a.kv_stride_tok, a.kv_stride_batch = 0, kv.stride(1), kv.stride(0)
        a.kv_rope_stride_page, a.kv_rope_stride_tok, a.kv_rope_stride_batch = 0, k_pe.stride(1), k_pe.stride(0)
        a.block_table = None
        a.block_table_stride = 0
        a.num_parts = num_parts
        a.cache_seqlens = seqlens.data_ptr()
        a.tile_sched = sched.data_ptr()
        a.num_splits = nsplits.data_ptr()
        a.lse = None
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel()
        # one split per sequence: the split-KV pass writes every output row, no combine
        fn = lib.mla_splitkv_fwd if self.splits == 1 else lib.mla_decode_fwd
        name = "mla_splitkv_fwd" if self.splits == 1 else "mla_decode_fwd"
        return a, ctypes.byref(a), fn, name, ws

    def __call__(self, q: torch.Tensor, q_pe: torch.Tensor, kv: torch.Tensor, k_pe: torch.Tensor,
                 output: Optional[torch.Tensor] = None):
        # A repeat call on the same tensors (the reference's timing loops, a serving loop) only
        # sets the output pointer and launches: the arguments were validated and filled when
        # the key was first seen.
        key = self._key(q, q_pe, kv, k_pe, output)
        prep = self._prepared if self._prepared is not None and self._prepared[0] == key else None
        if prep is None:
            prep = (key, self._prepare(q, q_pe, kv, k_pe, output))
            self._prepared = prep
        a, ref, fn, name, _ws = prep[1]
        ret = output is None
        if ret:
            output = torch.empty(self.batch, self.heads, DIM, dtype=q.dtype, device=q.device)
        a.out = output.data_ptr()
        a.o_stride_b, a.o_stride_s, a.o_stride_h = output.stride(0), 0, output.stride(1)
        st = prep[0][2]
        check(name, fn(ref, st))
        return output if ret else None
