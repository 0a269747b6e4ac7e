"""CPU restatement of the fp8 latent-cache format -- test infrastructure only.

The reference has no fp8 path: its design notes list an fp8 KV cache as unexplored
(docs/mla_decode_best_implementation.md:1693).  This file defines the format the fp8 decode
and the fp8 append implement, so that their results can be checked:

  * ``e4m3_decode`` / ``e4m3_encode`` -- the OCP 8-bit floating-point format E4M3 ("fn":
    bias 7, no infinities, 0x7F / 0xFF are NaN, largest finite value 448, subnormals down to
    2^-9) with round-to-nearest-even, as published in the OCP 8-bit Floating Point
    Specification (OFP8), rev. 1.0.
  * ``block_scale_exp`` -- the per-token, per-128-dim scale: the smallest power of two 2^k
    with amax <= 448 * 2^k, k clamped to [-126, 127], computed from the bits of the bf16
    amax (so the device computes the same k without a division); amax = 0 gives k = 0.
  * ``quantize_latent`` / ``dequantize_latent`` -- a token's 512 latent values become 512
    e4m3 codes of x / 2^k (k per 128-dim block) and 4 fp32 scales 2^k; the value of a code
    is e4m3(code) * 2^k, exact in fp32 and in bf16.
  * ``append_paged_fp8`` -- the paged append of ``append_paged`` (mla_ref.py) into the fp8
    page layout: latent [num_blocks, 64, 512] codes, scales [num_blocks, 4, 64] fp32 (one
    row of 64 token scales per 128-dim block), rope [num_blocks, 64, 64] in bf16.
  * ``dequantize_pages`` -- the bf16-equivalent [num_blocks, 64, 576] cache the fp8 decode
    must agree with; the decode oracle is then ``mla_ref.decode_paged`` on it.

Pinning (tests/test_oracle_fp8.py): ``e4m3_decode`` against the code table's closed forms and
torch's ``float8_e4m3fn`` view; ``e4m3_encode`` against torch's ``float8_e4m3fn`` cast
(a library routine, round-to-nearest-even) on every bf16 bit pattern in range, and the
scale rule against a float64 brute force.
"""
from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0
LATENT = 512
ROPE = 64
BLOCK = 128
NBLK = LATENT // BLOCK
PAGE = 64


def _e4m3_value(c: np.ndarray) -> np.ndarray:
    """The value of each code from its fields: sign, 4-bit exponent (bias 7), 3-bit mantissa;
    exponent 0 is subnormal (m/8 * 2^-6); S.1111.111 is NaN."""
    c = c.astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return (sign * val).astype(np.float32)


_E4M3_TABLE = _e4m3_value(np.arange(256))


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values (NaN for 0x7F / 0xFF), through the 256-entry table."""
    return _E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float values (|x| <= 448 after scaling) -> uint8 codes, round to nearest even.

    Values above 448 in magnitude saturate to 448 (the decode's inputs never reach them:
    the block scale keeps |x| / 2^k <= 448); NaN encodes as 0x7F.
    """
    v = np.asarray(x, dtype=np.float64)
    sign = (np.signbit(v)).astype(np.int32) << 7
    a = np.abs(v)
    # quantum of the binade (subnormal binade for a < 2^-6): 2^(e - 3), e >= -6
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(e, -6.0)
    q = np.exp2(e - 3.0)
    n = np.rint(a / q)                      # round half to even on exact float64 ratios
    r = n * q                               # rounded magnitude, may step into the next binade
    r = np.minimum(r, E4M3_MAX)
    r = np.where(np.isnan(r), 0.0, r)      # NaN gets its code below
    # encode r
    with np.errstate(divide="ignore"):
        re = np.floor(np.log2(np.where(r > 0, r, 1.0)))
    sub = r < 2.0 ** -6
    exp_field = np.where(sub, 0, re + 7).astype(np.int32)
    mant = np.where(sub, np.rint(r / 2.0 ** -9), np.rint((r / np.exp2(re) - 1.0) * 8)).astype(np.int32)
    code = sign | (exp_field << 3) | mant
    code = np.where(r == 0, sign, code)
    code = np.where(np.isnan(v), 0x7F, code)
    return code.astype(np.uint8)


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).contiguous().view(torch.int16).numpy().astype(np.int32) & 0xFFFF


def block_scale_exp(amax_bf16: torch.Tensor) -> np.ndarray:
    """k per block from the bf16 amax: smallest k with amax <= 448 * 2^k, clamped."""
    bits = bf16_bits(amax_bf16.abs())
    ef = (bits >> 7) & 0xFF
    mant = bits & 0x7F
    # amax = 1.mant * 2^(ef - 127); 448 = 1.75 * 2^8; 1.75 is mantissa 0x60
    k = (ef - 127) - 8 + (mant > 0x60).astype(np.int32)
    k = np.where(ef == 0, -126, k)          # zero or subnormal amax
    k = np.where(bits == 0, 0, k)
    return np.clip(k, -126, 127).astype(np.int32)


def quantize_latent(latent: torch.Tensor):
    """latent [n, 512] (bf16 values) -> (codes uint8 [n, 512], scales fp32 [n, 4])."""
    x = latent.to(torch.bfloat16).float()
    n = x.shape[0]
    blocks = x.reshape(n, NBLK, BLOCK)
    amax = blocks.abs().amax(-1).to(torch.bfloat16)       # exact: a max of bf16 values
    k = block_scale_exp(amax)                               # [n, 4]
    scaled = blocks.numpy().astype(np.float64) / np.exp2(k)[..., None]
    codes = e4m3_encode(scaled).reshape(n, LATENT)
    return codes, np.exp2(k).astype(np.float32)


def dequantize_latent(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """codes [n, 512], scales [n, 4] -> float32 [n, 512]."""
    n = codes.shape[0]
    v = e4m3_decode(codes).reshape(n, NBLK, BLOCK) * scales[..., None]
    return v.reshape(n, LATENT).astype(np.float32)


def append_paged_fp8(latent_pages: np.ndarray, scale_pages: np.ndarray, rope_pages: torch.Tensor,
                     block_table: torch.Tensor, cache_seqlens: torch.Tensor, kv_new: torch.Tensor):
    """Append kv_new [B, n_new, 576] (bf16) at positions L_b .. L_b + n_new - 1.

    latent_pages uint8 [nb, 64, 512], scale_pages float32 [nb, 4, 64], rope_pages bf16
    [nb, 64, 64] are updated copies; returns (latent, scales, rope, new_lens).  The page and
    row of a position are those of mla_ref.append_paged.
    """
    lat = latent_pages.copy()
    sc = scale_pages.copy()
    rope = rope_pages.clone()
    lens = cache_seqlens.clone()
    B, n_new, _ = kv_new.shape
    codes, scales = quantize_latent(kv_new[..., :LATENT].reshape(B * n_new, LATENT))
    codes = codes.reshape(B, n_new, LATENT)
    scales = scales.reshape(B, n_new, NBLK)
    for b in range(B):
        L = int(cache_seqlens[b])
        for t in range(n_new):
            pos = L + t
            pg = int(block_table[b, pos // PAGE])
            row = pos % PAGE
            lat[pg, row] = codes[b, t]
            sc[pg, :, row] = scales[b, t]
            rope[pg, row] = kv_new[b, t, LATENT:].to(rope.dtype)
        lens[b] = L + n_new
    return lat, sc, rope, lens


def dequantize_pages(latent_pages: np.ndarray, scale_pages: np.ndarray, rope_pages: torch.Tensor):
    """-> float32 [nb, 64, 1, 576]: the cache the fp8 decode is checked against."""
    nb = latent_pages.shape[0]
    scales = np.transpose(scale_pages, (0, 2, 1)).reshape(nb * PAGE, NBLK)
    lat = dequantize_latent(latent_pages.reshape(nb * PAGE, LATENT), scales)
    kv = torch.cat([torch.from_numpy(lat).reshape(nb, PAGE, LATENT), rope_pages.float()], -1)
    return kv.reshape(nb, PAGE, 1, LATENT + ROPE)


def quantize_pages(kv_cache: torch.Tensor):
    """bf16 cache [nb, 64, 1|-, 576] -> (latent codes [nb,64,512], scales [nb,4,64], rope)."""
    nb = kv_cache.shape[0]
    flat = kv_cache.reshape(nb * PAGE, LATENT + ROPE)
    codes, scales = quantize_latent(flat[:, :LATENT])
    lat = codes.reshape(nb, PAGE, LATENT)
    sc = np.ascontiguousarray(np.transpose(scales.reshape(nb, PAGE, NBLK), (0, 2, 1)))
    rope = flat[:, LATENT:].to(torch.bfloat16).reshape(nb, PAGE, ROPE).contiguous()
    return lat, sc, rope
