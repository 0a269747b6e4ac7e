"""GPU parity of the absorbed value projection with the combine fused into it
(``mla_combine_absorb``) against a float32 reference of the same product (the decode oracle's
output times W_UV per head, then W_O)."""
import sys

import pytest
import torch
import torch.nn.functional as F

from mlc_decode_amd import (flash_mla_with_kvcache, get_mla_metadata, mla_decode_absorbed,
                            prepare_w_uv)
from mlc_decode_amd.inputs import make_inputs
from oracle import mla_ref as R

from test_gpu_parity import small_cfg

pytestmark = pytest.mark.gpu

# v is rounded to bf16 (8 significant bits) and so is the merged row it is computed from (the
# decode's own output precision); with weights ~ N(0, 1/512) |v| reaches ~4 for one-key rows.
# Bar: max-abs error <= 2^-7 of the largest |v| (two bf16 roundings of the largest value), and
# cosine >= 0.9999 against the fp32 product of the fp32 oracle's rows.
V_RTOL = 2.0 ** -7
COS_MIN = 0.9999


def say(msg):
    print(f"[gpu-absorb] {msg}", flush=True)
    sys.stdout.flush()


def weights(H, dtype, seed, d_model=0):
    g = torch.Generator().manual_seed(seed)
    w_uv = (torch.randn(H, 512, 128, generator=g) * 512 ** -0.5).to(dtype)
    w_o = (torch.randn(H * 128, d_model, generator=g) * (H * 128) ** -0.5).to(dtype) if d_model else None
    return w_uv, w_o


def check_close(got, ref, atol, what):
    got = got.float().cpu()
    assert torch.isfinite(got).all(), f"{what}: non-finite"
    err = (got - ref).abs().max().item()
    assert err <= atol, f"{what}: max-abs {err}"
    if ref.abs().max() > 0:
        cos = F.cosine_similarity(got.flatten().double(), ref.flatten().double(), dim=0).item()
        assert cos >= COS_MIN, f"{what}: cosine {cos}"


# forced 12: 60 parts for 5 sequences, merged in the fused kernel's prologue; forced 40: 200
# parts (at least 16 per sequence), merged first by the combine kernel's dim-quarter form and
# read back by the projection (v bit-identical either way, checked below)
@pytest.mark.parametrize("H,s_q", [(16, 1), (64, 1), (128, 1), (128, 2)])
@pytest.mark.parametrize("forced", [0, 1, 3, 12, 40])
def test_absorb_matches_reference(gpu, H, s_q, forced):
    cfg = small_cfg(f"absorb_h{H}", 5, s_q, H, [0, 1, 100, 700, 3000])
    inp = make_inputs(cfg, seed=H + forced)
    w_uv, _ = weights(H, torch.bfloat16, H)
    d = inp.to("cuda")
    say(f"absorb H={H} s_q={s_q} forced={forced}")
    sched, splits = get_mla_metadata(d.cache_seqlens, s_q * H, 1, forced_splits=forced)
    v, lse = mla_decode_absorbed(d.q, d.kv_cache, d.block_table, d.cache_seqlens, sched, splits,
                                 prepare_w_uv(w_uv.cuda()), softmax_scale=inp.sm_scale, causal=True)
    torch.cuda.synchronize()
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens, inp.sm_scale, True)
    ref_v = torch.einsum("bshk,hkn->bshn", ref_o, w_uv.float())
    check_close(v, ref_v, V_RTOL * ref_v.abs().max().item(), f"v H={H} s_q={s_q} forced={forced}")
    # the fused merge is the combine kernel's (one shared routine): the rows are bit-identical,
    # so v differs from the fp32 product of the combine's output only by v's own rounding to
    # bf16 (half an ulp, <= 2^-8 |v|) and fp32 summation order (<= 2^-14 of sum |o_k w_kn|)
    out, lse2 = flash_mla_with_kvcache(d.q, d.kv_cache, d.block_table, d.cache_seqlens, 512, sched, splits,
                                       softmax_scale=inp.sm_scale, causal=True)
    o2 = out.float().cpu()
    v2 = torch.einsum("bshk,hkn->bshn", o2, w_uv.float())
    mag = torch.einsum("bshk,hkn->bshn", o2.abs(), w_uv.float().abs())
    vv = v.float().cpu()
    bad = (vv - v2).abs() > v2.abs() * 2.0 ** -8 + mag * 2.0 ** -14 + 1e-6
    assert not bad.any(), f"fused merge differs from combine at {bad.nonzero()[:4].tolist()}"
    assert torch.equal(lse.cpu(), lse2.cpu()), "fused lse differs from combine"


@pytest.mark.parametrize("forced", [0, 1])
def test_absorb_large_grid(gpu, forced):
    # 40 sequences x 2 queries: rows in several 16-row tiles, sequences of ragged lengths
    H, s_q, B = 128, 2, 40
    lens = [(37 * i * i + 5 * i) % 900 + 1 for i in range(B)]
    cfg = small_cfg("absorb_big", B, s_q, H, lens)
    inp = make_inputs(cfg, seed=21 + forced)
    w_uv, _ = weights(H, torch.bfloat16, 17)
    d = inp.to("cuda")
    say(f"absorb large grid forced={forced}")
    sched, splits = get_mla_metadata(d.cache_seqlens, s_q * H, 1, forced_splits=forced)
    v, lse = mla_decode_absorbed(d.q, d.kv_cache, d.block_table, d.cache_seqlens, sched, splits,
                                 prepare_w_uv(w_uv.cuda()), softmax_scale=inp.sm_scale, causal=True)
    out, lse2 = flash_mla_with_kvcache(d.q, d.kv_cache, d.block_table, d.cache_seqlens, 512, sched, splits,
                                       softmax_scale=inp.sm_scale, causal=True)
    torch.cuda.synchronize()
    ref_o, _ = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens, inp.sm_scale, True)
    ref_v = torch.einsum("bshk,hkn->bshn", ref_o, w_uv.float())
    check_close(v, ref_v, V_RTOL * ref_v.abs().max().item(), f"v large grid forced={forced}")
    o2 = out.float().cpu()
    v2 = torch.einsum("bshk,hkn->bshn", o2, w_uv.float())
    mag = torch.einsum("bshk,hkn->bshn", o2.abs(), w_uv.float().abs())
    bad = (v.float().cpu() - v2).abs() > v2.abs() * 2.0 ** -8 + mag * 2.0 ** -14 + 1e-6
    assert not bad.any(), f"fused merge differs from combine at {bad.nonzero()[:4].tolist()}"
    assert torch.equal(lse.cpu(), lse2.cpu())


def test_absorb_with_output_projection(gpu):
    H = 128
    cfg = small_cfg("absorb_wo", 4, 1, H, [64, 500, 1000, 4096])
    inp = make_inputs(cfg, seed=3)
    w_uv, w_o = weights(H, torch.bfloat16, 7, d_model=1024)
    d = inp.to("cuda")
    say("absorb + W_O")
    sched, splits = get_mla_metadata(d.cache_seqlens, H, 1)
    y, lse = mla_decode_absorbed(d.q, d.kv_cache, d.block_table, d.cache_seqlens, sched, splits,
                                 prepare_w_uv(w_uv.cuda()), w_o.cuda(), softmax_scale=inp.sm_scale, causal=True)
    torch.cuda.synchronize()
    ref_o, _ = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens, inp.sm_scale, True)
    ref_y = torch.einsum("bshk,hkn->bshn", ref_o, w_uv.float()).reshape(4, 1, H * 128) @ w_o.float()
    check_close(y, ref_y, 2 * V_RTOL * ref_y.abs().max().item(), "y = v W_O")


def test_absorb_fp16(gpu):
    H = 64
    cfg = small_cfg("absorb_f16", 3, 1, H, [33, 2000, 129], dtype=torch.float16)
    inp = make_inputs(cfg, seed=5)
    w_uv, _ = weights(H, torch.float16, 5)
    d = inp.to("cuda")
    say("absorb fp16")
    sched, splits = get_mla_metadata(d.cache_seqlens, H, 1, forced_splits=4)
    v, _ = mla_decode_absorbed(d.q, d.kv_cache, d.block_table, d.cache_seqlens, sched, splits,
                               prepare_w_uv(w_uv.cuda()), softmax_scale=inp.sm_scale, causal=True)
    torch.cuda.synchronize()
    ref_o, _ = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens, inp.sm_scale, True)
    ref_v = torch.einsum("bshk,hkn->bshn", ref_o, w_uv.float())
    check_close(v, ref_v, V_RTOL * ref_v.abs().max().item(), "v fp16")


def _fused_equals_combine(v, lse, out, lse2, w_uv, what):
    o2 = out.float().cpu()
    v2 = torch.einsum("bshk,hkn->bshn", o2, w_uv.float())
    mag = torch.einsum("bshk,hkn->bshn", o2.abs(), w_uv.float().abs())
    bad = (v.float().cpu() - v2).abs() > v2.abs() * 2.0 ** -8 + mag * 2.0 ** -14 + 1e-6
    assert not bad.any(), f"{what}: fused merge differs from combine at {bad.nonzero()[:4].tolist()}"
    assert torch.equal(lse.cpu(), lse2.cpu()), f"{what}: lse differs"


def test_absorb_fp8_cache(gpu):
    # the projection reads only the split partials: any cache format the decode takes works
    from mlc_decode_amd import quantize_kv_cache
    H = 128
    cfg = small_cfg("absorb_fp8", 4, 1, H, [5, 300, 1000, 2500])
    inp = make_inputs(cfg, seed=8)
    w_uv, _ = weights(H, torch.bfloat16, 8)
    d = inp.to("cuda")
    cache = quantize_kv_cache(d.kv_cache)
    say("absorb fp8 cache")
    sched, splits = get_mla_metadata(d.cache_seqlens, H, 1, forced_splits=3)
    v, lse = mla_decode_absorbed(d.q, cache, d.block_table, d.cache_seqlens, sched, splits,
                                 prepare_w_uv(w_uv.cuda()), softmax_scale=inp.sm_scale, causal=True)
    out, lse2 = flash_mla_with_kvcache(d.q, cache, d.block_table, d.cache_seqlens, 512, sched, splits,
                                       softmax_scale=inp.sm_scale, causal=True)
    torch.cuda.synchronize()
    _fused_equals_combine(v, lse, out, lse2, w_uv, "fp8")


def test_absorb_sparse(gpu):
    H, B, topk, nb = 64, 3, 700, 30
    g = torch.Generator().manual_seed(12)
    kv = torch.randn(nb, 64, 1, 576, generator=g).to(torch.bfloat16).cuda()
    q = torch.randn(B, 1, H, 576, generator=g).to(torch.bfloat16).cuda()
    idx = torch.randint(0, nb * 64, (B, 1, topk), generator=g, dtype=torch.int32)
    idx[:, :, ::7] = -1
    idx = idx.cuda()
    w_uv, _ = weights(H, torch.bfloat16, 12)
    lens = torch.zeros(B, dtype=torch.int32, device="cuda")
    say("absorb sparse")
    sched, splits = get_mla_metadata(lens, H, 1, topk=topk, forced_splits=2)
    v, lse = mla_decode_absorbed(q, kv, None, None, sched, splits, prepare_w_uv(w_uv.cuda()),
                                 softmax_scale=576 ** -0.5, indices=idx)
    out, lse2 = flash_mla_with_kvcache(q, kv, None, None, 512, sched, splits, softmax_scale=576 ** -0.5,
                                       indices=idx)
    torch.cuda.synchronize()
    _fused_equals_combine(v, lse, out, lse2, w_uv, "sparse")
    ref_o, _ = R.decode_sparse(q.cpu(), kv.cpu(), idx.cpu(), 576 ** -0.5)
    ref_v = torch.einsum("bshk,hkn->bshn", ref_o, w_uv.float())
    check_close(v, ref_v, V_RTOL * ref_v.abs().max().item(), "v sparse")


@pytest.mark.parametrize("H", [16, 128])
def test_absorb_long_single_sequence(gpu, H):
    """Batch 1 at 16K tokens under the default schedule (up to 256 splits of the one sequence):
    the merge runs in the combine kernel's dim-quarter form and the projection reads the merged
    rows; against the oracle and against the combine's own rows and lse."""
    cfg = small_cfg(f"absorb_long_h{H}", 1, 1, H, [16384])
    inp = make_inputs(cfg, seed=60 + H)
    w_uv, _ = weights(H, torch.bfloat16, 60 + H)
    d = inp.to("cuda")
    say(f"absorb long single sequence H={H}")
    sched, splits = get_mla_metadata(d.cache_seqlens, H, 1)
    assert splits[-1].item() > 64  # a long merge
    v, lse = mla_decode_absorbed(d.q, d.kv_cache, d.block_table, d.cache_seqlens, sched, splits,
                                 prepare_w_uv(w_uv.cuda()), softmax_scale=inp.sm_scale, causal=True)
    out, lse2 = flash_mla_with_kvcache(d.q, d.kv_cache, d.block_table, d.cache_seqlens, 512, sched, splits,
                                       softmax_scale=inp.sm_scale, causal=True)
    torch.cuda.synchronize()
    _fused_equals_combine(v, lse, out, lse2, w_uv, f"long H={H}")
    ref_o, _ = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens, inp.sm_scale, True)
    ref_v = torch.einsum("bshk,hkn->bshn", ref_o, w_uv.float())
    check_close(v, ref_v, V_RTOL * ref_v.abs().max().item(), f"v long H={H}")
