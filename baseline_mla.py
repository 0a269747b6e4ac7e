"""Drop-in ``baseline_mla`` for MI355X: the serial (one split per sequence) decode.

``_get_kernel`` returns the same HIP kernel as ``mla_decode`` with ``num_splits = 1``
(one workgroup walks a sequence's whole cache, the reference's T_b role,
baseline_mla.py:192-197).  ``ref_program`` is the reference's torch checker
(baseline_mla.py:167-191), evaluated in fp32 on the inputs' device; the decode path never
calls it.
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import torch  # noqa: E402

from mla_decode import _split_plan  # noqa: E402
from mlc_decode_amd.legacy import MlaKernel  # noqa: E402


def flashattn(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, block_N, block_H, num_split,
              softmax_scale):
    """Kernel with ``num_split`` page ranges per sequence (1 = serial)."""
    ns = _split_plan(seqlen_kv, max(1, int(num_split)), 64, False)[0]
    return MlaKernel(batch, heads, kv_head_num, seqlen_kv, dim, pe_dim, splits=ns,
                     config=dict(block_N=block_N, block_H=block_H, num_split=num_split),
                     sm_scale=softmax_scale)


def ref_program(q, q_pe, kv, k_pe):
    """softmax([q|q_pe] . [kv|k_pe]^T / sqrt(dim + pe_dim)) . kv, in fp32, returned in q's
    dtype.  Shapes: q [B, H, dim], q_pe [B, H, pe], kv [B, L, Hk, dim], k_pe [B, L, Hk, pe]."""
    dim, pe_dim = q.shape[-1], q_pe.shape[-1]
    b, h = q.shape[0], q.shape[1]
    hk = kv.shape[2]
    g = h // hk
    query = torch.cat([q, q_pe], dim=-1).float().reshape(b, hk, g, dim + pe_dim)
    key = torch.cat([kv, k_pe], dim=-1).float().permute(0, 2, 1, 3)        # [b, hk, L, d]
    scores = torch.matmul(query, key.transpose(-1, -2).contiguous()) / (dim + pe_dim) ** 0.5
    attn = torch.softmax(scores, dim=-1)
    out = torch.matmul(attn, kv.float().permute(0, 2, 1, 3).contiguous())  # [b, hk, g, dim]
    return out.reshape(b, h, dim).to(q.dtype)


def _get_kernel(batch, heads, kv_heads, kv_ctx, dim, pe_dim):
    softmax_scale = (dim + pe_dim) ** -0.5
    return MlaKernel(batch, heads, kv_heads, kv_ctx, dim, pe_dim, splits=1, sm_scale=softmax_scale)


def _bench_ms(kernel, args, warmup=10, rep=50):
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
    return s.elapsed_time(e) / rep


def _randn_inputs(batch, heads, kv_heads, kv_ctx, dim, pe_dim, dtype=torch.float16):
    g = torch.Generator(device="cpu").manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(dtype).cuda()  # noqa: E731
    return (mk(batch, heads, dim), mk(batch, heads, pe_dim), mk(batch, kv_ctx, kv_heads, dim),
            mk(batch, kv_ctx, kv_heads, pe_dim))


def main(batch=1, heads=128, kv_heads=1, kv_ctx=8192, dim=512, pe_dim=64):
    """Check against ref_program, then time the serial kernel (reference :200-218)."""
    qk_flops = 2 * batch * heads * kv_ctx * (dim + pe_dim)
    pv_flops = 2 * batch * heads * kv_ctx * dim
    kernel = _get_kernel(batch, heads, kv_heads, kv_ctx, dim, pe_dim)
    args = _randn_inputs(batch, heads, kv_heads, kv_ctx, dim, pe_dim)
    out = torch.empty_like(args[0])
    kernel(*args, out)
    ref = ref_program(*args)
    # fp16 output of an fp32-accumulated decode: compare at fp16 resolution
    torch.testing.assert_close(out.float(), ref.float(), rtol=2e-3, atol=2e-3)
    latency = _bench_ms(kernel, args, warmup=50)
    tflops = (qk_flops + pv_flops) / latency * 1e-9
    print(f"Latency: {latency} ms")
    print(f"TFlops: {tflops} TFlops")
    return latency, tflops


def run_regression_perf(batch=1, heads=128, kv_heads=1, kv_ctx=8192, dim=512, pe_dim=64):
    kernel = _get_kernel(batch, heads, kv_heads, kv_ctx, dim, pe_dim)
    args = _randn_inputs(batch, heads, kv_heads, kv_ctx, dim, pe_dim)
    out = torch.empty_like(args[0])
    kernel(*args, out)
    torch.testing.assert_close(out.float(), ref_program(*args).float(), rtol=2e-3, atol=2e-3)
    return _bench_ms(kernel, args)


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--json", type=str, default=None, help="JSON file with test cases")
    parser.add_argument("--no-json", action="store_true", help="Skip JSON mode, use single-case CLI args")
    parser.add_argument("--batch", type=int, default=132, help="batch size")
    parser.add_argument("--heads", type=int, default=128, help="q heads number")
    parser.add_argument("--kv_heads", type=int, default=1, help="kv heads number")
    parser.add_argument("--kv_ctx", type=int, default=8192, help="kv context length")
    parser.add_argument("--dim", type=int, default=512, help="head dim")
    parser.add_argument("--pe_dim", type=int, default=64, help="pe head dim")
    args = parser.parse_args()
    if args.no_json or args.json is None:
        main(args.batch, args.heads, args.kv_heads, args.kv_ctx, args.dim, args.pe_dim)
    else:
        with open(args.json) as f:
            cases = json.load(f)
        passed = failed = 0
        csv_path = os.path.splitext(args.json)[0] + "_results.csv"
        fields = ["case_id", "batch", "heads", "kv_heads", "kv_ctx", "dim", "pe_dim",
                  "latency_ms", "tflops", "status"]
        with open(csv_path, "w", newline="") as fh:
            writer = csv.DictWriter(fh, fieldnames=fields)
            writer.writeheader()
            for c in cases:
                row = {k: c.get(k, d) for k, d in (("case_id", "?"), ("batch", 1), ("heads", 16),
                                                    ("kv_heads", 1), ("kv_ctx", 8192), ("dim", 512),
                                                    ("pe_dim", 64))}
                print(f"[Case {row['case_id']}] batch={row['batch']}, kv_ctx={row['kv_ctx']}")
                try:
                    lat, tfl = main(row["batch"], row["heads"], row["kv_heads"], row["kv_ctx"],
                                    row["dim"], row["pe_dim"])
                    row.update(latency_ms=round(lat, 6), tflops=round(tfl, 4), status="PASS")
                    passed += 1
                    print(f"[Case {row['case_id']}] PASS  latency={lat:.4f}ms  tflops={tfl:.4f}")
                except Exception as e:  # noqa: BLE001 - every failure is reported per case
                    err_msg = str(e).split("\n")[0]
                    row.update(latency_ms=-1, tflops=-1, status=f"FAIL: {err_msg}")
                    failed += 1
                    print(f"[Case {row['case_id']}] FAIL: {err_msg}")
                writer.writerow(row)
        print(f"\n=== Summary: {passed}/{len(cases)} passed, {failed}/{len(cases)} failed ===")
        print(f"CSV saved to: {csv_path}")
