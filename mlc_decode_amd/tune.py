"""Split-policy sweep per context length, written into the reference's two tuning records.

Interface kept from the reference (scripts/tune_best.py): the command-line flags
(``--kv-ctx``, ``--batch``, ``--heads``, ``--kv-heads``, ``--dim``, ``--pe-dim``, ``--warmup``,
``--rep``) and the two JSON files it maintains, ``mla_best_configs.json`` (context -> fastest
config with its ``latency_us``; read by scripts/mla_prof.py:30-35) and ``mla_tune_all.json``
(context -> every measured candidate).  Everything else is this module's own design:

* candidates come from ``mla_decode.mla_autotune_configs`` (the balanced schedule and forced
  per-sequence split counts) and are built with ``build_kernel_from_config``;
* inputs: one seeded CPU generator draws the fused query ``[B, H, dim + pe_dim]`` and the fused
  contiguous cache ``[B, ctx, kv_heads, dim + pe_dim]`` (fp16, N(0, 0.1^2): the reference's
  distribution and dtype), and the latent / rope halves are views of them, which the C ABI
  takes as they are;
* each candidate is timed by ``mlc_decode_amd.timing`` (clock settling, then ``--windows``
  windows of ``--rep`` back-to-back calls after ``--warmup`` untimed ones, HIP events on the
  launch stream) and its median window is recorded, together with the spread;
* a candidate that fails (the library rejects it, a launch error) is logged and left out of
  the records, so the rest of the sweep goes on;
* both files are rewritten after every context (atomically, through a temporary file), so an
  interrupted sweep keeps what it measured.

    python -m mlc_decode_amd.tune --kv-ctx 2048 4096 8192 [--out-dir DIR] [--windows 3]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BEST_FILE = "mla_best_configs.json"
ALL_FILE = "mla_tune_all.json"


@dataclass
class Shape:
    batch: int
    heads: int
    kv_heads: int
    dim: int
    pe_dim: int

    def inputs(self, ctx: int, seed: int = 0):
        """(q, q_pe, kv, k_pe, out) on the GPU: halves of two fused fp16 tensors."""
        import torch
        g = torch.Generator("cpu").manual_seed(seed)
        width = self.dim + self.pe_dim
        qf = (torch.randn(self.batch, self.heads, width, generator=g) * 0.1).half().cuda()
        cache = (torch.randn(self.batch, ctx, self.kv_heads, width, generator=g) * 0.1).half().cuda()
        out = torch.zeros(self.batch, self.heads, self.dim, dtype=torch.float16, device="cuda")
        return (qf[..., :self.dim], qf[..., self.dim:], cache[..., :self.dim], cache[..., self.dim:], out)


@dataclass
class Measurement:
    config: dict
    windows_us: List[float] = field(default_factory=list)
    error: Optional[str] = None

    @property
    def ok(self) -> bool:
        return self.error is None and bool(self.windows_us)

    @property
    def us(self) -> float:
        return statistics.median(self.windows_us)

    def row(self) -> dict:
        """The record entry: the candidate's own keys plus its median latency."""
        return {**self.config, "latency_us": round(self.us, 3)}

    def describe(self) -> str:
        ns = self.config.get("num_split")
        label = "balanced" if ns is None else f"forced {ns}"
        if not self.ok:
            return f"{label:>10}  FAILED  {self.error}"
        lo, hi = min(self.windows_us), max(self.windows_us)
        return f"{label:>10}  {self.us:9.2f} us  (windows {lo:.2f} .. {hi:.2f})"


def time_candidate(kernel: Callable, call_args: tuple, warmup: int, rep: int, windows: int) -> List[float]:
    """µs per call in each of ``windows`` timing windows of ``rep`` calls."""
    import torch

    from .timing import settle_clocks, time_gpu
    stream = torch.cuda.current_stream()
    run = lambda: kernel(*call_args)  # noqa: E731
    settle_clocks(run, stream, seconds=0.1)
    return [time_gpu(run, rep, warmup if w == 0 else 0, stream) * 1e3 for w in range(windows)]


def sweep_context(shape: Shape, ctx: int, warmup: int, rep: int, windows: int,
                  log: Callable[[str], None] = print) -> List[Measurement]:
    """Every candidate of one context length, measured in the order the configs list them."""
    if REPO not in sys.path:
        sys.path.insert(0, REPO)
    from mla_decode import build_kernel_from_config, mla_autotune_configs

    call_args = shape.inputs(ctx)
    configs = mla_autotune_configs(shape.batch, shape.heads, shape.kv_heads, ctx, shape.dim, shape.pe_dim)
    log(f"context {ctx}: {len(configs)} candidates (batch {shape.batch}, heads {shape.heads})")
    results = []
    for cfg in configs:
        m = Measurement(dict(cfg))
        t0 = time.perf_counter()
        try:
            kernel = build_kernel_from_config(shape.batch, shape.heads, shape.kv_heads, ctx, shape.dim,
                                              shape.pe_dim, cfg)
            m.windows_us = time_candidate(kernel, call_args, warmup, rep, windows)
        except (RuntimeError, ValueError) as exc:  # a rejected config or a failed launch
            m.error = f"{type(exc).__name__}: {exc}"
        results.append(m)
        log(f"  {m.describe()}  [{time.perf_counter() - t0:.1f} s]")
    return results


class TuneRecords:
    """The two JSON records in ``directory``, merged with what they already hold."""

    def __init__(self, directory: str):
        self.directory = directory
        self.best = self._read(BEST_FILE)
        self.all = self._read(ALL_FILE)

    def _read(self, name: str) -> dict:
        path = os.path.join(self.directory, name)
        if not os.path.exists(path):
            return {}
        with open(path) as f:
            return json.load(f)

    def update(self, ctx: int, results: List[Measurement]) -> Optional[dict]:
        good = [m for m in results if m.ok]
        if not good:
            return None
        fastest = min(good, key=lambda m: m.us)
        self.best[str(ctx)] = fastest.row()
        self.all[str(ctx)] = [m.row() for m in good]
        return self.best[str(ctx)]

    def save(self) -> List[str]:
        os.makedirs(self.directory, exist_ok=True)
        written = []
        for name, data in ((BEST_FILE, self.best), (ALL_FILE, self.all)):
            path = os.path.join(self.directory, name)
            tmp = path + ".partial"
            with open(tmp, "w") as f:
                json.dump(data, f, indent=2, sort_keys=True)
                f.write("\n")
            os.replace(tmp, path)
            written.append(path)
        return written


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description="time every split policy per context length and record the fastest")
    # the reference's flags
    ap.add_argument("--kv-ctx", type=int, nargs="+", required=True, help="context lengths to sweep")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--heads", type=int, default=16)
    ap.add_argument("--kv-heads", type=int, default=1)
    ap.add_argument("--dim", type=int, default=512)
    ap.add_argument("--pe-dim", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=20, help="untimed calls before the first window")
    ap.add_argument("--rep", type=int, default=50, help="timed calls per window")
    # this module's own
    ap.add_argument("--windows", type=int, default=3, help="timing windows per candidate (median kept)")
    ap.add_argument("--out-dir", default=REPO, help="directory of the two JSON records")
    return ap.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    shape = Shape(args.batch, args.heads, args.kv_heads, args.dim, args.pe_dim)
    records = TuneRecords(args.out_dir)
    say = lambda s: print(s, flush=True)  # noqa: E731
    for ctx in args.kv_ctx:
        results = sweep_context(shape, ctx, args.warmup, args.rep, max(1, args.windows), log=say)
        chosen = records.update(ctx, results)
        say(f"  fastest: {chosen}" if chosen else "  no candidate ran; context left out of the records")
        for path in records.save():
            say(f"  wrote {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
