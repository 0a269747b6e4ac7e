"""Pins of the fp8 latent-cache oracle (oracle/mla_fp8_ref.py) -- CPU only."""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import mla_fp8_ref as F
from oracle import mla_ref as R


def test_e4m3_decode_matches_torch_view():
    codes = np.arange(256, dtype=np.uint8)
    ours = F.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    # closed forms of the table
    assert ours[0x38] == 1.0 and ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9
    assert ours[0x08] == 2.0 ** -6 and ours[0xB8] == -1.0 and np.isnan(ours[0x7F])


def test_e4m3_encode_matches_torch_cast_on_every_bf16_in_range():
    bits = np.arange(1 << 16, dtype=np.int32).astype(np.uint16).view(np.int16)
    x = torch.from_numpy(bits).view(torch.bfloat16).float()
    finite = torch.isfinite(x) & (x.abs() <= F.E4M3_MAX)
    x = x[finite]
    ours = F.e4m3_encode(x.numpy())
    ref = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e4m3_encode_ties_and_saturation():
    # ties go to the even code; beyond 448 saturates (the encoder's inputs never get there)
    xs = np.array([1.0625, 1.1875, 2.0 ** -10, 1.5 * 2.0 ** -9, 464.0, -500.0, np.nan])
    got = F.e4m3_encode(xs)
    assert got.tolist() == [0x38, 0x3A, 0x00, 0x02, 0x7E, 0xFE, 0x7F]


def _k_bruteforce(a: float) -> int:
    if a == 0:
        return 0
    r = Fraction(a) / 448
    k = math.ceil(math.log2(float(r))) + 2
    while Fraction(2) ** (k - 1) >= r:
        k -= 1
    return max(-126, min(127, k))


def test_block_scale_rule_against_bruteforce():
    vals = [0.0, 448.0, 449.0, 447.0, 7 * 2.0 ** 6, 7 * 2.0 ** -20, 7 * 2.0 ** -20 * 1.0078125,
            1.0, 3.0e38, 1e-40, 2.0 ** -130, 224.0, 225.0]
    rng = np.random.default_rng(0)
    vals += list((rng.standard_normal(2000) * np.exp2(rng.integers(-60, 60, 2000))).astype(np.float32))
    t = torch.tensor(vals, dtype=torch.float32).to(torch.bfloat16)
    ks = F.block_scale_exp(t)
    for v, k in zip(t.float().tolist(), ks.tolist()):
        assert k == _k_bruteforce(abs(v)), (v, k)


def test_quantize_error_bounds_and_scale_range():
    torch.manual_seed(0)
    x = (torch.randn(256, 512) * torch.exp2(torch.randint(-8, 8, (256, 1)).float())).to(torch.bfloat16)
    codes, scales = F.quantize_latent(x)
    deq = F.dequantize_latent(codes, scales)
    xf = x.float().numpy()
    blocks = np.abs(xf).reshape(256, 4, 128).max(-1)
    ratio = blocks / scales
    assert np.all((ratio > 224) & (ratio <= 448))           # scale is the tightest power of two
    assert np.all(np.log2(scales) == np.round(np.log2(scales)))
    s_full = np.repeat(scales, 128, axis=1)
    normal = np.abs(xf) / s_full >= 2.0 ** -6
    err = np.abs(deq - xf)
    assert np.all(err[normal] <= np.abs(xf[normal]) * 2.0 ** -4)   # half an ulp of a 3-bit mantissa
    assert np.all(err[~normal] <= s_full[~normal] * 2.0 ** -10)    # half the subnormal step
    # values that are already codes times the scale come back exactly
    again, sc2 = F.quantize_latent(torch.from_numpy(deq).to(torch.bfloat16))
    assert np.array_equal(F.dequantize_latent(again, sc2), deq)


def test_append_fp8_equals_quantized_bf16_append():
    torch.manual_seed(1)
    nb, B, n_new = 12, 3, 2
    kv = torch.randn(nb, 64, 1, 576).to(torch.bfloat16)
    table = torch.randperm(nb).reshape(B, 4).to(torch.int32)
    lens = torch.tensor([5, 63, 128], dtype=torch.int32)
    new = torch.randn(B, n_new, 576).to(torch.bfloat16)
    lat, sc, rope = F.quantize_pages(kv)
    lat2, sc2, rope2, lens2 = F.append_paged_fp8(lat, sc, rope, table, lens, new)
    kv_ref, lens_ref, _ = R.append_paged(kv, table, lens, new)
    lat3, sc3, rope3 = F.quantize_pages(kv_ref)
    assert torch.equal(lens2, lens_ref)
    assert np.array_equal(lat2, lat3) and np.array_equal(sc2, sc3) and torch.equal(rope2, rope3)


def test_dequantized_pages_round_trip_layout():
    torch.manual_seed(2)
    kv = torch.randn(3, 64, 1, 576).to(torch.bfloat16)
    lat, sc, rope = F.quantize_pages(kv)
    deq = F.dequantize_pages(lat, sc, rope)
    assert deq.shape == (3, 64, 1, 576)
    assert torch.equal(deq[..., 512:], kv[..., 512:].float())
    # token (page 1, row 5), block 2: the scale of that block scales its codes
    k = sc[1, 2, 5]
    codes = lat[1, 5, 256:384]
    assert np.array_equal(deq[1, 5, 0, 256:384].numpy(), F.e4m3_decode(codes) * k)
