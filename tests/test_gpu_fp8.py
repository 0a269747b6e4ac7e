"""GPU parity of the fp8 latent cache: the quantizing append against the fp8 oracle
(bit-exact), and the fp8 decode against the fp32 oracle decode of the dequantised cache (the
same bar as the bf16 path: max-abs <= 1e-2, cosine >= 0.99999, LSE within 1e-3)."""
import math
import random
import sys

import numpy as np
import pytest
import torch

from mlc_decode_amd import (Fp8KVCache, flash_mla_with_kvcache, fp8_kv_cache, get_mla_metadata,
                            kv_append, mla_decode_with_kvcache, quantize_kv_cache)
from mlc_decode_amd.inputs import CONFIGS, MlaConfig, make_inputs
from oracle import mla_fp8_ref as F8
from oracle import mla_ref as R

from test_gpu_parity import assert_parity, small_cfg

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-fp8] {msg}", flush=True)
    sys.stdout.flush()


def varied_cache(nb, seed):
    """bf16 pages whose 128-dim blocks span many scale exponents, with zero and tiny blocks."""
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn(nb, 64, 1, 576, generator=g)
    mag = torch.exp2(torch.randint(-20, 20, (nb, 64, 1, 4), generator=g).float())
    mag = mag * (1 + torch.rand(nb, 64, 1, 4, generator=g))
    kv[..., :512] = (kv[..., :512].reshape(nb, 64, 1, 4, 128) * mag[..., None]).reshape(nb, 64, 1, 512)
    kv[0, 3, 0, 128:256] = 0.0                       # a zero block (scale 1)
    kv[0, 4, 0, :128] = 1e-38                        # subnormal-range block
    kv[0, 5, 0, 384:] = 448.0                        # exactly 448 * 2^0
    kv[0, 6, 0, 384:] = -3.0e38                      # near the bf16 maximum
    return kv.to(torch.bfloat16)


def to_gpu_fp8(lat, sc, rope):
    return Fp8KVCache(torch.from_numpy(lat).cuda(), torch.from_numpy(sc).cuda(), rope.cuda())


def assert_fp8_equal(c: Fp8KVCache, lat, sc, rope, what):
    got_lat = c.latent.cpu().numpy()
    got_sc = c.scale.cpu().numpy()
    bad = np.argwhere(got_lat != lat)
    assert bad.size == 0, f"{what}: {len(bad)} codes differ, first {bad[:4].tolist()} " \
                          f"got {got_lat[tuple(bad[0])]} want {lat[tuple(bad[0])]}"
    assert np.array_equal(got_sc, sc), f"{what}: scales differ"
    assert torch.equal(c.rope.cpu(), rope), f"{what}: rope differs"


def test_quantize_cache_matches_oracle(gpu):
    kv = varied_cache(6, 0)
    say("quantize_kv_cache 6 pages")
    got = quantize_kv_cache(kv.cuda())
    torch.cuda.synchronize()
    lat, sc, rope = F8.quantize_pages(kv)
    assert_fp8_equal(got, lat, sc, rope, "quantize_kv_cache")


@pytest.mark.parametrize("n_new", [1, 2, 5])
def test_fp8_append_matches_oracle(gpu, n_new):
    torch.manual_seed(10 + n_new)
    nb, B = 16, 4
    base = varied_cache(nb, n_new)
    lat, sc, rope = F8.quantize_pages(base)
    table = torch.randperm(nb).reshape(B, 4).to(torch.int32)
    lens = torch.tensor([0, 63, 64, 130], dtype=torch.int32)
    new = varied_cache(B, 100 + n_new).reshape(B, 64, 576)[:, :n_new].contiguous()
    cache = to_gpu_fp8(lat, sc, rope)
    lens_d = lens.cuda()
    say(f"fp8 append n_new={n_new}")
    kv_append(new.cuda(), cache, table.cuda(), lens_d)
    torch.cuda.synchronize()
    lat2, sc2, rope2, lens2 = F8.append_paged_fp8(lat, sc, rope, table, lens, new)
    assert torch.equal(lens_d.cpu(), lens2)
    assert_fp8_equal(cache, lat2, sc2, rope2, f"append n_new={n_new}")


def fp8_inputs(cfg, seed, quantize_on_gpu=False):
    """(inputs, fp8 cache on the GPU, dequantised fp32 cache for the oracle).  Large caches
    are quantised on the GPU (its quantiser is checked bit-exact against the oracle above)
    and only dequantised on the CPU, a table lookup."""
    inp = make_inputs(cfg, seed=seed)
    if quantize_on_gpu:
        cache = quantize_kv_cache(inp.kv_cache.cuda())
        torch.cuda.synchronize()
        deq = F8.dequantize_pages(cache.latent.cpu().numpy(), cache.scale.cpu().numpy(), cache.rope.cpu())
        return inp, cache, deq
    lat, sc, rope = F8.quantize_pages(inp.kv_cache)
    deq = F8.dequantize_pages(lat, sc, rope)
    return inp, to_gpu_fp8(lat, sc, rope), deq


def check_fp8(inp, cache, deq, rows=None, num_splits=None, what=""):
    d = inp.to("cuda")
    out, lse = mla_decode_with_kvcache(d.q, cache, d.block_table, d.cache_seqlens, num_splits=num_splits,
                                       sm_scale=inp.sm_scale, causal=inp.causal)
    torch.cuda.synchronize()
    idx = torch.arange(inp.q.shape[0]) if rows is None else torch.tensor(rows)
    ref_out, ref_lse = R.decode_paged(inp.q[idx], deq, inp.block_table[idx], inp.cache_seqlens[idx],
                                      inp.sm_scale, inp.causal)
    assert_parity(out[idx.cuda()], lse[idx.cuda()], ref_out, ref_lse, what)
    return out, lse


TAILS = [0, 1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 1000]


@pytest.mark.parametrize("H", [16, 32, 64, 128])
def test_fp8_tails_all_head_counts(gpu, H):
    cfg = small_cfg(f"fp8_tails_h{H}", len(TAILS), 1, H, TAILS)
    inp, cache, deq = fp8_inputs(cfg, seed=H)
    say(f"fp8 tails H={H}")
    check_fp8(inp, cache, deq, what=f"fp8 tails H={H}")


@pytest.mark.parametrize("H,s_q", [(16, 2), (64, 2), (128, 2)])
def test_fp8_causal_mtp(gpu, H, s_q):
    cfg = small_cfg(f"fp8_mtp_h{H}", 4, s_q, H, [2, 65, 700, 2049])
    inp, cache, deq = fp8_inputs(cfg, seed=7 * H)
    say(f"fp8 causal H={H} s_q={s_q}")
    check_fp8(inp, cache, deq, what=f"fp8 causal H={H}")


@pytest.mark.parametrize("forced", [1, 3, 8])
def test_fp8_forced_splits(gpu, forced):
    cfg = small_cfg("fp8_splits", 3, 1, 16, [1, 700, 5000])
    inp, cache, deq = fp8_inputs(cfg, seed=forced)
    say(f"fp8 forced splits {forced}")
    check_fp8(inp, cache, deq, num_splits=forced, what=f"fp8 splits {forced}")


@pytest.mark.parametrize("name", ["C3", "C5"])
def test_fp8_benchmark_configs_sampled(gpu, name):
    cfg = CONFIGS[name]
    if cfg.dtype != torch.bfloat16:
        cfg = MlaConfig(cfg.name, batch=cfg.batch, s_q=cfg.s_q, heads=cfg.heads, dtype=torch.bfloat16,
                        sigma=cfg.sigma, seqlen=cfg.seqlen, seqlen_groups=cfg.seqlen_groups,
                        causal=cfg.causal, num_splits=cfg.num_splits)
    inp, cache, deq = fp8_inputs(cfg, seed=0, quantize_on_gpu=True)
    rows = sorted(random.Random(1).sample(range(cfg.batch), 6))
    say(f"fp8 {name} rows {rows}")
    out, lse = check_fp8(inp, cache, deq, rows=rows, what=f"fp8 {name}")
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()


def test_fp8_matches_bf16_kernel_on_dequantized_cache(gpu):
    # the dequantised values are exact in bf16: the two kernels see the same numbers
    cfg = small_cfg("fp8_vs_bf16", 5, 1, 16, [1, 64, 333, 1024, 4097])
    inp, cache, deq = fp8_inputs(cfg, seed=3)
    d = inp.to("cuda")
    say("fp8 vs bf16 kernel")
    o8, l8 = mla_decode_with_kvcache(d.q, cache, d.block_table, d.cache_seqlens, sm_scale=inp.sm_scale)
    o16, l16 = mla_decode_with_kvcache(d.q, deq.to(torch.bfloat16).cuda(), d.block_table, d.cache_seqlens,
                                       sm_scale=inp.sm_scale)
    torch.cuda.synchronize()
    assert (o8.float() - o16.float()).abs().max().item() <= 4e-3
    assert (l8 - l16).abs().max().item() <= 1e-4


def test_fp8_append_then_decode(gpu):
    # decode after appending new tokens through the quantizing append equals the oracle
    torch.manual_seed(5)
    nb, B, n_new = 24, 3, 3
    cfg = small_cfg("fp8_app", B, 1, 16, [5, 200, 700])
    inp = make_inputs(cfg, seed=11)
    lat, sc, rope = F8.quantize_pages(inp.kv_cache)
    cache = to_gpu_fp8(lat, sc, rope)
    new = torch.randn(B, n_new, 576).to(torch.bfloat16)
    lens = inp.cache_seqlens.clone().cuda()
    table = inp.block_table.cuda()
    say("fp8 append then decode")
    kv_append(new.cuda(), cache, table, lens)
    sched, splits = get_mla_metadata(lens, 16, 1)
    out, lse = flash_mla_with_kvcache(inp.q.cuda(), cache, table, lens, 512, sched, splits,
                                      softmax_scale=inp.sm_scale, causal=True)
    torch.cuda.synchronize()
    lat2, sc2, rope2, lens2 = F8.append_paged_fp8(lat, sc, rope, inp.block_table, inp.cache_seqlens, new)
    deq = F8.dequantize_pages(lat2, sc2, rope2)
    ref_out, ref_lse = R.decode_paged(inp.q, deq, inp.block_table, lens2, inp.sm_scale, True)
    assert_parity(out, lse, ref_out, ref_lse, "fp8 append then decode")
