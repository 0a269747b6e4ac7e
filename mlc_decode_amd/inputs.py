"""Seeded synthetic inputs for the five benchmark configurations.

Protocol (one CPU generator seeded with 0, fixed draw order):
  1. per-sequence cache lengths (ragged configs) via ``torch.randint(lo, hi + 1, ...)``;
  2. the block table: ``torch.randperm(total_pages)`` handed out row by row, unused slots 0
     (identity table for the plumbing config);
  3. ``q = randn(B, s_q, H, 576) * sigma``;
  4. ``kv = randn(total_pages, 64, 1, 576) * sigma``;
  5. cast to the config dtype on the CPU, then copied to the device, so a CPU checker and
     the GPU see identical bits.
The paged layout follows the reference's FlashMLA call (handmade/bench_metax_flashmla.py:22-30).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch

PAGE = 64
D_QK = 576
D_V = 512


@dataclass
class MlaConfig:
    name: str
    batch: int
    s_q: int
    heads: int
    dtype: torch.dtype
    sigma: float = 1.0
    seqlen: Optional[int] = None            # uniform length
    seqlen_groups: List[tuple] = field(default_factory=list)  # [(count, lo, hi) | (count, L)]
    identity_table: bool = False
    causal: bool = True
    num_splits: Optional[int] = None        # None = scheduler

    @property
    def sm_scale(self) -> float:
        return D_QK ** -0.5


CONFIGS = {
    "C1": MlaConfig("C1", batch=1, s_q=1, heads=16, dtype=torch.bfloat16, seqlen=1024,
                    identity_table=True, num_splits=1),
    "C2": MlaConfig("C2", batch=64, s_q=1, heads=128, dtype=torch.bfloat16, seqlen=4096),
    "C3": MlaConfig("C3", batch=128, s_q=1, heads=16, dtype=torch.bfloat16,
                    seqlen_groups=[(128, 256, 8192)]),
    # num_splits >= 8: the combine merges many partial O / LSE tiles per row
    "C4": MlaConfig("C4", batch=32, s_q=2, heads=128, dtype=torch.bfloat16, seqlen=16384,
                    num_splits=8),
    "C5": MlaConfig("C5", batch=132, s_q=1, heads=64, dtype=torch.float16, sigma=0.5,
                    seqlen_groups=[(1, 16384), (31, 2048, 8192), (100, 1, 128)]),
}


@dataclass
class MlaInputs:
    q: torch.Tensor            # [B, s_q, H, 576]
    kv_cache: torch.Tensor     # [num_pages, 64, 1, 576]
    block_table: torch.Tensor  # [B, max_pages] int32
    cache_seqlens: torch.Tensor  # [B] int32
    sm_scale: float
    causal: bool

    def to(self, device) -> "MlaInputs":
        return MlaInputs(self.q.to(device), self.kv_cache.to(device), self.block_table.to(device),
                         self.cache_seqlens.to(device), self.sm_scale, self.causal)


def draw_lengths(cfg: MlaConfig, g: torch.Generator) -> torch.Tensor:
    if cfg.seqlen is not None:
        return torch.full((cfg.batch,), cfg.seqlen, dtype=torch.int64)
    parts = []
    for grp in cfg.seqlen_groups:
        if len(grp) == 2:
            parts.append(torch.full((grp[0],), grp[1], dtype=torch.int64))
        else:
            n, lo, hi = grp
            parts.append(torch.randint(lo, hi + 1, (n,), generator=g, dtype=torch.int64))
    lengths = torch.cat(parts)
    assert lengths.numel() == cfg.batch
    return lengths


def make_inputs(cfg: MlaConfig, seed: int = 0, device: Optional[str] = None,
                lengths: Optional[torch.Tensor] = None) -> MlaInputs:
    """Inputs of ``cfg`` under the seeded protocol (``lengths`` overrides step 1)."""
    g = torch.Generator("cpu").manual_seed(seed)
    if lengths is None:
        lengths = draw_lengths(cfg, g)
    lengths = lengths.to(torch.int64)
    pages = (lengths + PAGE - 1) // PAGE
    total = int(pages.sum())
    max_pages = max(int(pages.max()), 1)
    if cfg.identity_table:
        order = torch.arange(total, dtype=torch.int64)
    else:
        order = torch.randperm(total, generator=g)
    table = torch.zeros(cfg.batch, max_pages, dtype=torch.int32)
    off = 0
    for b in range(cfg.batch):
        n = int(pages[b])
        table[b, :n] = order[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(cfg.batch, cfg.s_q, cfg.heads, D_QK, generator=g) * cfg.sigma
    kv = torch.randn(max(total, 1), PAGE, 1, D_QK, generator=g) * cfg.sigma
    inp = MlaInputs(q.to(cfg.dtype), kv.to(cfg.dtype), table, lengths.to(torch.int32),
                    cfg.sm_scale, cfg.causal)
    return inp.to(device) if device is not None else inp


def algorithmic_bytes(lengths, batch: int, s_q: int, heads: int, elem: int = 2) -> int:
    """HBM bytes one decode must move: KV once, q in, out and lse out."""
    total_l = int(torch.as_tensor(lengths).to(torch.int64).sum())
    return (total_l * D_QK * elem + batch * s_q * heads * D_QK * elem
            + batch * s_q * heads * D_V * elem + batch * s_q * heads * 4)


def algorithmic_flops(lengths, s_q: int, heads: int, causal: bool = True) -> int:
    """MFMA flops of one decode: QK (576) + PV (512) per visible (row, key) pair."""
    tot = 0
    for L in torch.as_tensor(lengths).tolist():
        for i in range(s_q):
            vis = L - (s_q - 1 - i) if causal else L
            tot += max(vis, 0)
    return 2 * heads * tot * (D_QK + D_V)
