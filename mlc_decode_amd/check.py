"""Correctness + timing check of the drop-in decode path against a float32 torch decode.

The command line and the output columns are those of the reference's ``scripts/check_mla.py``
(:47-92): per context length, the kernel's time, the float32 torch decode's time, the speed-up,
the max-abs error and the cosine similarity.

Usage:
    python -m mlc_decode_amd.check --kv-ctx 16384
    python -m mlc_decode_amd.check --kv-ctx 2048 4096 8192 16384 32768 65536

The kernel is the drop-in ``mla_decode._get_kernel`` path (contiguous fp16 layout).  Inputs are
drawn on the CPU from one seeded generator (N(0, 0.1^2)) and copied to the GPU; times come from
``mlc_decode_amd.timing`` (HIP events on the launch stream after a clock-settling run).
"""
import argparse
import os
import sys
import traceback

import torch

from .timing import settle_clocks, time_gpu


def torch_ref(q, q_pe, kv, k_pe, batch, heads, kv_heads, kv_ctx, dim, pe_dim):
    """float32 decode on q's device: for every KV head j and its query group,
    ``softmax([q | q_pe] . [kv | k_pe]^T / sqrt(dim + pe_dim)) . kv``.

    Shapes as the reference's kernels take them: q [B, H, dim], q_pe [B, H, pe_dim],
    kv [B, L, Hk, dim], k_pe [B, L, Hk, pe_dim] -> [B, H, dim] float32.  Written with
    batched fp32 products over (batch, KV head) pairs; right operands are made contiguous.
    """
    group = heads // kv_heads
    scale = 1.0 / float(dim + pe_dim) ** 0.5
    # (batch, kv head) pairs as the batch of one bmm
    qf = torch.cat([q, q_pe], dim=-1).float().reshape(batch * kv_heads, group, dim + pe_dim)
    keys = torch.cat([kv, k_pe], dim=-1).float().transpose(1, 2).reshape(batch * kv_heads, kv_ctx, dim + pe_dim)
    vals = kv.float().transpose(1, 2).reshape(batch * kv_heads, kv_ctx, dim).contiguous()
    logits = torch.bmm(qf, keys.transpose(1, 2).contiguous()) * scale
    weights = torch.softmax(logits, dim=-1)
    return torch.bmm(weights, vals).reshape(batch, heads, dim)


def _inputs(b, h, kh, ctx, d, pd, seed):
    g = torch.Generator().manual_seed(seed)
    draw = lambda *s: (torch.randn(*s, generator=g) * 0.1).to(torch.float16).cuda()  # noqa: E731
    return draw(b, h, d), draw(b, h, pd), draw(b, ctx, kh, d), draw(b, ctx, kh, pd)


def check_one(ctx, b=1, h=16, kh=1, d=512, pd=64, warmup=10, rep=50, seed=0):
    """One context length -> dict(our_us, torch_us, max_abs_err, cos_sim)."""
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    from mla_decode import _get_kernel

    q, q_pe, kv, k_pe = _inputs(b, h, kh, ctx, d, pd, seed)
    out = torch.empty_like(q)
    kernel = _get_kernel(b, h, kh, ctx, d, pd)
    run = lambda: kernel(q, q_pe, kv, k_pe, out)  # noqa: E731
    ref_run = lambda: torch_ref(q, q_pe, kv, k_pe, b, h, kh, ctx, d, pd)  # noqa: E731
    settle_clocks(run, seconds=0.05)
    our_us = time_gpu(run, rep, warmup) * 1e3
    torch_us = time_gpu(ref_run, rep, warmup) * 1e3
    ref = ref_run()
    o = out.float()
    err = (o - ref).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(o.flatten().double(), ref.flatten().double(), dim=0).item()
    return {"our_us": our_us, "torch_us": torch_us, "max_abs_err": err, "cos_sim": cos}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--kv-ctx", type=int, nargs="+", default=[16384])
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--heads", type=int, default=16)
    ap.add_argument("--kv-heads", type=int, default=1)
    ap.add_argument("--dim", type=int, default=512)
    ap.add_argument("--pe-dim", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--rep", type=int, default=50)
    args = ap.parse_args(argv)

    shape = (args.batch, args.heads, args.kv_heads, args.dim, args.pe_dim)
    print(f"device: {torch.cuda.get_device_name(0)}")
    header = ("kv_ctx", "Our(us)", "Torch(us)", "vsTorch", "max_abs_err", "cos_sim")
    widths = (8, 10, 10, 9, 12, 9)
    print("  ".join(f"{t:>{w}}" for t, w in zip(header, widths)))
    print("-" * 70)
    rows = []
    for ctx in args.kv_ctx:
        b, h, kh, d, pd = shape
        try:
            r = check_one(ctx, b, h, kh, d, pd, args.warmup, args.rep)
        except Exception as exc:  # noqa: BLE001 - a failing context is reported, the rest still run
            print(f"{ctx:>8}  FAIL {type(exc).__name__}: {str(exc)[:120]}")
            traceback.print_exc()
        else:
            rows.append((ctx, r))
            cells = (f"{ctx}", f"{r['our_us']:.2f}", f"{r['torch_us']:.2f}",
                     f"{r['torch_us'] / r['our_us']:.2f}x", f"{r['max_abs_err']:.6f}", f"{r['cos_sim']:.6f}")
            print("  ".join(f"{c:>{w}}" for c, w in zip(cells, widths)), flush=True)
        torch.cuda.empty_cache()
    return rows


if __name__ == "__main__":
    main()
