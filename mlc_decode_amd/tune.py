"""Per-context candidate timing, the MI355X counterpart of the reference's
scripts/tune_best.py (same flags, same two outputs).

Every candidate of ``mla_decode.mla_autotune_configs`` (the balanced schedule and the forced
per-sequence split counts) is built with ``build_kernel_from_config`` and timed with HIP
events (``--warmup`` untimed calls, then ``--rep`` timed back-to-back calls) on the
reference's inputs: fp16 ``randn * 0.1`` query, rope and contiguous latent cache, seed 0
(scripts/tune_best.py:71-77).  Writes

    <out-dir>/mla_best_configs.json   the fastest candidate per context, with latency_us
    <out-dir>/mla_tune_all.json       every candidate's measured latency per context

merging into existing files as the reference does (scripts/tune_best.py:62-63,101-108).

    python -m mlc_decode_amd.tune --kv-ctx 2048 4096 8192 [--out-dir DIR]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_json(path: str) -> dict:
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f)
    return {}


def time_us(kernel, call_args, warmup: int, rep: int) -> float:
    """Mean µs per call over ``rep`` back-to-back calls, after ``warmup`` untimed ones."""
    import torch

    from .timing import time_gpu
    stream = torch.cuda.current_stream()
    return time_gpu(lambda: kernel(*call_args), rep, warmup, stream) * 1000.0


def tune_context(ctx: int, batch: int, heads: int, kv_heads: int, dim: int, pe_dim: int,
                 warmup: int, rep: int, log=print):
    """(best row, all rows) for one context length."""
    import torch

    if REPO not in sys.path:
        sys.path.insert(0, REPO)
    from mla_decode import build_kernel_from_config, mla_autotune_configs

    torch.manual_seed(0)
    q = torch.randn(batch, heads, dim, dtype=torch.float16, device="cuda") * 0.1
    q_pe = torch.randn(batch, heads, pe_dim, dtype=torch.float16, device="cuda") * 0.1
    kv = torch.randn(batch, ctx, kv_heads, dim, dtype=torch.float16, device="cuda") * 0.1
    k_pe = torch.randn(batch, ctx, kv_heads, pe_dim, dtype=torch.float16, device="cuda") * 0.1
    out = torch.zeros(batch, heads, dim, dtype=torch.float16, device="cuda")
    call_args = (q, q_pe, kv, k_pe, out)

    configs = mla_autotune_configs(batch, heads, kv_heads, ctx, dim, pe_dim)
    log(f"\n=== kv_ctx={ctx}  {len(configs)} configs ===")
    rows, best = [], None
    for i, cfg in enumerate(configs):
        t0 = time.time()
        kernel = build_kernel_from_config(batch, heads, kv_heads, ctx, dim, pe_dim, cfg)
        us = time_us(kernel, call_args, warmup, rep)
        row = dict(cfg, latency_us=round(us, 3))
        rows.append(row)
        tag = ""
        if best is None or us < best["latency_us"]:
            best, tag = row, "  <-- best"
        ns = "sched" if cfg["num_split"] is None else f"{cfg['num_split']:5d}"
        log(f"  [{i:2d}] ns={ns} spread={int(cfg['spread'])} block_N={cfg['block_N']} "
            f"us={us:8.2f} ({time.time() - t0:4.1f}s){tag}")
    return best, rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--kv-ctx", type=int, nargs="+", required=True)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--heads", type=int, default=16)
    ap.add_argument("--kv-heads", type=int, default=1)
    ap.add_argument("--dim", type=int, default=512)
    ap.add_argument("--pe-dim", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rep", type=int, default=50)
    ap.add_argument("--out-dir", default=REPO, help="where the two JSON files are written")
    args = ap.parse_args(argv)

    best_path = os.path.join(args.out_dir, "mla_best_configs.json")
    all_path = os.path.join(args.out_dir, "mla_tune_all.json")
    best_all, tune_all = load_json(best_path), load_json(all_path)
    for ctx in args.kv_ctx:
        best, rows = tune_context(ctx, args.batch, args.heads, args.kv_heads, args.dim, args.pe_dim,
                                  args.warmup, args.rep, log=lambda s: print(s, flush=True))
        best_all[str(ctx)] = best
        tune_all[str(ctx)] = rows
        print(f"  => best: {best}", flush=True)
    os.makedirs(args.out_dir, exist_ok=True)
    with open(best_path, "w") as f:
        json.dump(best_all, f, indent=2, sort_keys=True)
    with open(all_path, "w") as f:
        json.dump(tune_all, f, indent=2, sort_keys=True)
    print(f"\nsaved {best_path}\nsaved {all_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
