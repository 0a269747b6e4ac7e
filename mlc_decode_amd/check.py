"""Correctness + timing check of the decode kernel against a float32 torch reference, with the
command line and output columns of the reference's ``scripts/check_mla.py`` (:47-92):
kernel time, torch time, speed-up, max-abs error and cosine similarity per context length.

Usage:
    python -m mlc_decode_amd.check --kv-ctx 16384
    python -m mlc_decode_amd.check --kv-ctx 2048 4096 8192 16384 32768 65536

The kernel is the drop-in ``mla_decode._get_kernel`` path (contiguous fp16 layout); the
reference is the float32 softmax(Q K^T / sqrt(576)) V of ``scripts/check_mla.py:21-32``, computed
on the GPU with plain matmuls (no batched low-precision products).
"""
import argparse
import os
import sys
import traceback

import torch


def torch_ref(q, q_pe, kv, k_pe, batch, heads, kv_heads, kv_ctx, dim, pe_dim):
    """float32 MLA decode: out[b, h] = softmax([q, q_pe] . [kv, k_pe]^T * (dim + pe_dim)^-1/2) kv."""
    group_num = heads // kv_heads
    q_main = q.reshape(batch, kv_heads, group_num, dim).float()
    q_pos = q_pe.reshape(batch, kv_heads, group_num, pe_dim).float()
    kv_main = kv.permute(0, 2, 1, 3).float().contiguous()      # [b, kv_heads, ctx, dim]
    k_pos = k_pe.permute(0, 2, 1, 3).float().contiguous()
    query = torch.cat([q_main, q_pos], dim=-1)                  # [b, kv_heads, g, 576]
    key_t = torch.cat([kv_main, k_pos], dim=-1).transpose(-1, -2).contiguous()
    scores = torch.matmul(query, key_t) * ((dim + pe_dim) ** -0.5)
    out = torch.matmul(torch.softmax(scores, dim=-1), kv_main)  # [b, kv_heads, g, dim]
    return out.reshape(batch, heads, dim)


def bench(fn, warmup=10, rep=50):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(rep):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / rep * 1000


def check_one(ctx, b=1, h=16, kh=1, d=512, pd=64, warmup=10, rep=50, seed=0):
    """One context length -> dict(our_us, torch_us, max_abs_err, cos_sim)."""
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    from mla_decode import _get_kernel

    torch.manual_seed(seed)
    q = torch.randn(b, h, d, dtype=torch.float16, device="cuda") * 0.1
    q_pe = torch.randn(b, h, pd, dtype=torch.float16, device="cuda") * 0.1
    kv = torch.randn(b, ctx, kh, d, dtype=torch.float16, device="cuda") * 0.1
    k_pe = torch.randn(b, ctx, kh, pd, dtype=torch.float16, device="cuda") * 0.1
    out = torch.empty_like(q)
    kernel = _get_kernel(b, h, kh, ctx, d, pd)
    our_us = bench(lambda: kernel(q, q_pe, kv, k_pe, out), warmup=warmup, rep=rep)
    ref = torch_ref(q, q_pe, kv, k_pe, b, h, kh, ctx, d, pd)
    torch_us = bench(lambda: torch_ref(q, q_pe, kv, k_pe, b, h, kh, ctx, d, pd), warmup=warmup, rep=rep)
    err = (out.float() - ref).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(out.float().flatten(), ref.flatten(), dim=0).item()
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

    b, h, kh, d, pd = args.batch, args.heads, args.kv_heads, args.dim, args.pe_dim
    print(f"device: {torch.cuda.get_device_name(0)}")
    print(f"{'kv_ctx':>8}  {'Our(us)':>10}  {'Torch(us)':>10}  {'vsTorch':>9}  {'max_abs_err':>12}  {'cos_sim':>9}")
    print("-" * 70)
    rows = []
    for ctx in args.kv_ctx:
        try:
            r = check_one(ctx, b, h, kh, d, pd, args.warmup, args.rep)
            rows.append((ctx, r))
            print(f"{ctx:>8}  {r['our_us']:>10.2f}  {r['torch_us']:>10.2f}  {r['torch_us'] / r['our_us']:>8.2f}x  "
                  f"{r['max_abs_err']:>12.6f}  {r['cos_sim']:>9.6f}", flush=True)
        except Exception as e:  # noqa: BLE001 - report and continue, as the reference script does
            print(f"{ctx:>8}  FAIL {type(e).__name__}: {str(e)[:120]}")
            traceback.print_exc()
        torch.cuda.empty_cache()
    return rows


if __name__ == "__main__":
    main()
