"""GPU parity of the sparse (top-k) decode against the fp32 oracle (``decode_sparse``), with the
same bar as the dense path (max-abs <= 1e-2, cosine >= 0.99999, LSE within 1e-3)."""
import sys

import pytest
import torch

from mlc_decode_amd import flash_mla_with_kvcache, get_mla_metadata
from mlc_decode_amd.inputs import make_inputs
from oracle import mla_ref as R

from test_gpu_parity import assert_parity, small_cfg

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-sparse] {msg}", flush=True)
    sys.stdout.flush()


def sparse_case(B, H, topk, nb, seed, dtype=torch.bfloat16, invalid=0.1, dup=0.05):
    g = torch.Generator().manual_seed(seed)
    kv = (torch.randn(nb, 64, 1, 576, generator=g)).to(dtype)
    q = (torch.randn(B, 1, H, 576, generator=g)).to(dtype)
    idx = torch.randint(0, nb * 64, (B, 1, topk), generator=g, dtype=torch.int32)
    r = torch.rand(B, 1, topk, generator=g)
    idx[r < invalid] = -1                                   # no key
    idx[(r >= invalid) & (r < invalid + 0.01)] = nb * 64 + 5  # past the pool: no key
    if topk > 1:                                            # repeated keys count twice
        d = torch.rand(B, 1, topk, generator=g) < dup
        idx[:, :, 1:][d[:, :, 1:]] = idx[:, :, :1].expand(-1, -1, topk - 1)[d[:, :, 1:]]
    return q, kv, idx


def run_sparse(q, kv, idx, scale=576 ** -0.5, forced=0):
    B, _, H, _ = q.shape
    topk = idx.shape[-1]
    dummy_lens = torch.zeros(B, dtype=torch.int32, device="cuda")
    sched, splits = get_mla_metadata(dummy_lens, H, 1, topk=topk, forced_splits=forced)
    out, lse = flash_mla_with_kvcache(q.cuda(), kv.cuda(), None, None, 512, sched, splits,
                                      softmax_scale=scale, indices=idx.cuda())
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("H", [16, 32, 64, 128])
@pytest.mark.parametrize("topk", [1, 31, 100, 2048])
def test_sparse_matches_oracle(gpu, H, topk):
    q, kv, idx = sparse_case(3, H, topk, nb=40, seed=H * 7 + topk)
    say(f"sparse H={H} topk={topk}")
    out, lse = run_sparse(q, kv, idx)
    ref_o, ref_l = R.decode_sparse(q, kv, idx, 576 ** -0.5)
    assert_parity(out, lse, ref_o, ref_l, f"sparse H={H} topk={topk}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("forced", [1, 4])
def test_sparse_dtypes_and_splits(gpu, dtype, forced):
    q, kv, idx = sparse_case(4, 16, 777, nb=30, seed=11, dtype=dtype)
    say(f"sparse {dtype} forced={forced}")
    out, lse = run_sparse(q, kv, idx, forced=forced)
    ref_o, ref_l = R.decode_sparse(q, kv, idx, 576 ** -0.5)
    assert_parity(out, lse, ref_o, ref_l, f"sparse {dtype} forced={forced}")


def test_sparse_all_invalid_rows(gpu):
    q, kv, idx = sparse_case(2, 16, 64, nb=4, seed=5)
    idx[1] = -1
    say("sparse all-invalid row")
    out, lse = run_sparse(q, kv, idx)
    assert torch.all(out[1] == 0) and torch.all(lse[1] == float("-inf"))
    ref_o, ref_l = R.decode_sparse(q, kv, idx, 576 ** -0.5)
    assert_parity(out, lse, ref_o, ref_l, "sparse all-invalid")


def test_sparse_with_dense_indices_equals_dense_kernel(gpu):
    cfg = small_cfg("sparse_dense", 4, 1, 64, [1, 65, 900, 2000])
    inp = make_inputs(cfg, seed=9)
    idx = R.dense_indices(inp.block_table, inp.cache_seqlens, 2048).reshape(4, 1, 2048)
    d = inp.to("cuda")
    say("sparse vs dense")
    so, sl = run_sparse(inp.q, inp.kv_cache, idx, inp.sm_scale)
    sched, splits = get_mla_metadata(d.cache_seqlens, 64, 1)
    do, dl = flash_mla_with_kvcache(d.q, d.kv_cache, d.block_table, d.cache_seqlens, 512, sched, splits,
                                    softmax_scale=inp.sm_scale, causal=True)
    torch.cuda.synchronize()
    assert (so.float() - do.float()).abs().max().item() <= 4e-3
    assert (sl - dl).abs().max().item() <= 1e-4
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens, inp.sm_scale)
    assert_parity(so, sl, ref_o, ref_l, "sparse dense-order")


@pytest.mark.parametrize("H", [16, 32, 64, 128])
def test_sparse_fp8_cache(gpu, H):
    # the top-k decode over the fp8 latent cache: the fp32 oracle of the dequantised pool, and
    # the sparse kernel on the dequantised (bf16-exact) pool
    from mlc_decode_amd import Fp8KVCache
    from oracle import mla_fp8_ref as F8
    q, kv, idx = sparse_case(3, H, 333, nb=24, seed=H + 1)
    lat, sc, rope = F8.quantize_pages(kv)
    deq = F8.dequantize_pages(lat, sc, rope)
    cache = Fp8KVCache(torch.from_numpy(lat).cuda(), torch.from_numpy(sc).cuda(), rope.cuda())
    say(f"sparse fp8 H={H}")
    dummy = torch.zeros(3, dtype=torch.int32, device="cuda")
    sched, splits = get_mla_metadata(dummy, H, 1, topk=333)
    out, lse = flash_mla_with_kvcache(q.cuda(), cache, None, None, 512, sched, splits,
                                      softmax_scale=576 ** -0.5, indices=idx.cuda())
    torch.cuda.synchronize()
    ref_o, ref_l = R.decode_sparse(q, deq, idx, 576 ** -0.5)
    assert_parity(out, lse, ref_o, ref_l, f"sparse fp8 H={H}")
    o16, l16 = run_sparse(q, deq.to(torch.bfloat16), idx)
    assert (out.float() - o16.float()).abs().max().item() <= 4e-3
    assert (lse - l16).abs().max().item() <= 1e-4
