"""Writes tests/golden/mla_cases.npz: small MLA decode cases with float64 expected outputs.

Expected values come from torch's scaled_dot_product_attention evaluated in float64 on the
gathered pages (a library routine, independent of oracle/mla_ref.py) and, for the LSE,
from torch.logsumexp in float64.  Inputs are drawn in bf16/fp16 and stored as their raw
16-bit patterns, so a test rebuilds the identical low-precision tensors; expected values are
stored as float32.

Run from the repository root:  python tests/golden/make_fixtures.py
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
PAGE, D, DV = 64, 576, 512

CASES = [
    # name, B, s_q, H, lengths, dtype, sigma, causal
    ("h16_l1", 1, 1, 16, [1], torch.bfloat16, 1.0, True),
    ("h16_tails", 3, 1, 16, [63, 65, 129], torch.bfloat16, 1.0, True),
    ("h16_sq2_causal", 3, 2, 16, [1, 2, 97], torch.bfloat16, 1.0, True),
    ("h64_fp16_ragged", 3, 1, 64, [5, 64, 100], torch.float16, 0.5, True),
    ("h128_sq2", 1, 2, 128, [130], torch.bfloat16, 1.0, True),
    ("h16_sq2_noncausal", 2, 2, 16, [40, 70], torch.float16, 1.0, False),
]


def expected(q, kv, table, lengths, scale, causal):
    B, s_q, H, _ = q.shape
    out = np.zeros((B, s_q, H, DV))
    lse = np.full((B, H, s_q), -np.inf)
    for b in range(B):
        L = lengths[b]
        n = (L + PAGE - 1) // PAGE
        k = kv[table[b, :n].long(), :, 0, :].reshape(-1, D)[:L].double()
        for i in range(s_q):
            vis = L - (s_q - 1 - i) if causal else L
            if vis <= 0:
                continue
            qq = q[b, i].double().unsqueeze(0)                    # [1, H, D]
            kk = k[:vis].unsqueeze(0).unsqueeze(0).expand(1, H, vis, D)
            vv = k[:vis, :DV].unsqueeze(0).unsqueeze(0).expand(1, H, vis, DV)
            o = F.scaled_dot_product_attention(qq.unsqueeze(2), kk, vv, scale=scale)  # [1,H,1,DV]
            out[b, i] = o[0, :, 0].numpy()
            lse[b, :, i] = torch.logsumexp(qq[0] @ k[:vis].t() * scale, -1).numpy()
    return out, lse


def main():
    g = torch.Generator("cpu").manual_seed(1234)
    arrays = {}
    for name, B, s_q, H, lengths, dtype, sigma, causal in CASES:
        pages = [(L + PAGE - 1) // PAGE for L in lengths]
        total = sum(pages)
        perm = torch.randperm(total, generator=g)
        table = torch.zeros(B, max(pages), dtype=torch.int32)
        off = 0
        for b, n in enumerate(pages):
            table[b, :n] = perm[off:off + n].to(torch.int32)
            off += n
        q = (torch.randn(B, s_q, H, D, generator=g) * sigma).to(dtype)
        kv = (torch.randn(total, PAGE, 1, D, generator=g) * sigma).to(dtype)
        scale = D ** -0.5
        out, lse = expected(q, kv, table, lengths, scale, causal)
        arrays[f"{name}.q"] = q.view(torch.int16).numpy()
        arrays[f"{name}.kv"] = kv.view(torch.int16).numpy()
        arrays[f"{name}.table"] = table.numpy()
        arrays[f"{name}.lengths"] = np.array(lengths, dtype=np.int32)
        arrays[f"{name}.meta"] = np.array([s_q, H, 0 if dtype == torch.bfloat16 else 1, int(causal)],
                                          dtype=np.int32)
        arrays[f"{name}.out"] = out.astype(np.float32)
        arrays[f"{name}.lse"] = lse.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "mla_cases.npz"), **arrays)
    print("wrote", sorted({k.split('.')[0] for k in arrays}))


if __name__ == "__main__":
    main()
