"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on identical inputs.

Bar: output max-abs error <= 1e-2 and cosine >= 0.99999 against the
fp32 oracle, LSE within 1e-3; rows with no visible key must give out == 0, lse == -inf.
Full-size benchmark configs are checked on a sample of their sequences (oracle cost) plus
whole-output properties.
"""
import math
import random
import sys

import pytest
import torch
import torch.nn.functional as F

from mlc_decode_amd import (MlaKernel, flash_mla_with_kvcache, get_mla_metadata, kv_append,
                            get_mla_metadata_host, merge_partials, mla_decode_with_kvcache)
from mlc_decode_amd.inputs import CONFIGS, MlaConfig, make_inputs
from oracle import mla_ref as R

pytestmark = pytest.mark.gpu

OUT_ATOL = 1e-2
COS_MIN = 0.99999
LSE_ATOL = 1e-3


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def assert_parity(out, lse, ref_out, ref_lse, what=""):
    o = out.float().cpu()
    r = ref_out.float()
    assert torch.isfinite(o).all(), f"{what}: non-finite output"
    err = (o - r).abs().max().item()
    assert err <= OUT_ATOL, f"{what}: max-abs {err}"
    if r.abs().max() > 0:
        cos = F.cosine_similarity(o.flatten().double(), r.flatten().double(), dim=0).item()
        assert cos >= COS_MIN, f"{what}: cosine {cos}"
    if lse is not None:
        lg = lse.float().cpu()
        fin = torch.isfinite(ref_lse)
        assert torch.equal(torch.isfinite(lg), fin), f"{what}: lse finiteness differs"
        assert torch.all(lg[~fin] == -math.inf), f"{what}: empty rows must have lse = -inf"
        if fin.any():
            lerr = (lg[fin] - ref_lse[fin]).abs().max().item()
            assert lerr <= LSE_ATOL, f"{what}: lse err {lerr}"


def run_paged(inp, device, num_splits=None):
    d = inp.to(device)
    out, lse = mla_decode_with_kvcache(d.q, d.kv_cache, d.block_table, d.cache_seqlens,
                                       num_splits=num_splits, sm_scale=inp.sm_scale, causal=inp.causal)
    torch.cuda.synchronize()
    return out, lse


def oracle_rows(inp, rows):
    """Oracle on a subset of sequences (indices `rows`)."""
    idx = torch.tensor(rows)
    return R.decode_paged(inp.q[idx], inp.kv_cache, inp.block_table[idx], inp.cache_seqlens[idx],
                          inp.sm_scale, inp.causal)


def small_cfg(name, B, s_q, H, lengths, dtype=torch.bfloat16, sigma=1.0, causal=True):
    return MlaConfig(name, batch=B, s_q=s_q, heads=H, dtype=dtype, sigma=sigma, causal=causal,
                     seqlen_groups=[(1, L) for L in lengths])


# ---------------------------------------------------------------- small exhaustive cases
TAILS = [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 1000]


@pytest.mark.parametrize("H", [16, 32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_tails_all_head_counts(gpu, H, dtype):
    cfg = small_cfg(f"tails_h{H}", len(TAILS), 1, H, TAILS, dtype)
    inp = make_inputs(cfg, seed=H)
    for ns in (None, 1, 3):
        say(f"tails H={H} dtype={dtype} num_splits={ns}")
        out, lse = run_paged(inp, gpu, ns)
        ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                      inp.sm_scale, inp.causal)
        assert_parity(out, lse, ref_o, ref_l, f"H={H} ns={ns}")


@pytest.mark.parametrize("H, s_q", [(40, 1), (48, 2), (96, 1), (40, 2), (80, 2)])
def test_head_counts_off_the_row_tile(gpu, H, s_q):
    """Row counts s_q*H that are not a multiple of the wide kernel's 64- or 128-row workgroup
    (padding rows), and head blocks whose rows span both query tokens: the general
    (row-by-row) store path of the epilogue, for direct outputs and for split partials."""
    lengths = [1, 33, 64, 65, 700, 2100]
    cfg = small_cfg(f"odd_h{H}_sq{s_q}", len(lengths), s_q, H, lengths)
    inp = make_inputs(cfg, seed=H + s_q)
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, inp.causal)
    for ns in (None, 1, 3):
        say(f"odd heads H={H} s_q={s_q} num_splits={ns}")
        out, lse = run_paged(inp, gpu, ns)
        assert_parity(out, lse, ref_o, ref_l, f"H={H} s_q={s_q} ns={ns}")


_RANDOM_HEADS = [1, 3, 8, 16, 24, 31, 40, 48, 64, 72, 96, 128, 136, 160]


@pytest.mark.parametrize("case", range(24))
def test_random_shapes(gpu, case):
    """Seeded random decodes across every kernel variant and grid form: head counts on and
    off the 16/32/64/128-row tiles (several head blocks above 128 rows), s_q 1 and 2, empty,
    one-token and page-straddling lengths, bf16 and fp16, the scheduler and forced splits."""
    rnd = random.Random(1000 + case)
    H = rnd.choice(_RANDOM_HEADS)
    s_q = rnd.choice([1, 1, 2])
    B = rnd.randint(1, 24)
    lengths = [rnd.choice([0, 1, 31, 64, 65, rnd.randint(1, 600), rnd.randint(600, 2600)]) for _ in range(B)]
    if max(lengths) == 0:
        lengths[0] = 17
    dtype = rnd.choice([torch.bfloat16, torch.float16])
    ns = rnd.choice([None, None, 1, rnd.randint(2, 6)])
    cfg = small_cfg(f"rand{case}", B, s_q, H, lengths, dtype)
    inp = make_inputs(cfg, seed=case)
    say(f"random case {case}: B={B} s_q={s_q} H={H} dtype={dtype} num_splits={ns} lengths={lengths}")
    out, lse = run_paged(inp, gpu, ns)
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, inp.causal)
    assert_parity(out, lse, ref_o, ref_l, f"random case {case}")


@pytest.mark.parametrize("H", [16, 64, 128])
def test_causal_two_queries(gpu, H):
    lengths = [1, 2, 33, 64, 65, 300]
    cfg = small_cfg(f"sq2_h{H}", len(lengths), 2, H, lengths)
    inp = make_inputs(cfg, seed=7)
    for ns in (None, 2):
        say(f"causal s_q=2 H={H} num_splits={ns}")
        out, lse = run_paged(inp, gpu, ns)
        ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                      inp.sm_scale, True)
        assert_parity(out, lse, ref_o, ref_l, f"sq2 H={H} ns={ns}")
    # L = 1: query 0 sees no key
    assert torch.all(out[0, 0].float() == 0)


def test_non_causal_two_queries(gpu):
    cfg = small_cfg("sq2_nc", 3, 2, 16, [5, 64, 200], causal=False)
    inp = make_inputs(cfg, seed=8)
    say("non-causal s_q=2")
    out, lse = run_paged(inp, gpu)
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, False)
    assert_parity(out, lse, ref_o, ref_l, "non-causal")


def test_empty_sequence_and_nan_padding(gpu):
    lengths = [0, 37, 1, 64, 130]
    cfg = small_cfg("edge", len(lengths), 1, 16, lengths)
    inp = make_inputs(cfg, seed=9)
    # poison every cache row past each sequence end, and unused table slots
    for b, L in enumerate(lengths):
        n = R.pages_of(L)
        if n and L % 64:
            inp.kv_cache[inp.block_table[b, n - 1].long(), L % 64:] = float("nan")
        inp.block_table[b, n:] = 1 << 30
    say("empty sequence + NaN padding")
    out, lse = run_paged(inp, gpu, 1)
    good = torch.tensor(lengths) > 0
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, True)
    assert_parity(out, lse, ref_o, ref_l, "edge")
    assert torch.all(out[~good].float() == 0) and torch.all(lse[~good].cpu() == -math.inf)


@pytest.mark.parametrize("H,s_q,splits", [(16, 1, None), (16, 1, 1), (128, 1, None), (64, 2, 3)])
def test_length_past_block_table_width(gpu, H, s_q, splits):
    """A cache_seqlens entry longer than the block table's row (64 * width tokens) is cut to
    the row: no column at or past the width is read, and the status word is raised.  The
    table is a view of the first P columns of a wider tensor whose later columns name pages
    full of NaN, so a read past the width would poison the output; the last sequence is the
    over-long one too, where a read past the row would leave the allocation."""
    P = 6
    lengths = [64 * P + 100, 64 * P, 200, 64 * P + 1]
    B = len(lengths)
    cfg = small_cfg(f"width_h{H}", B, s_q, H, [min(L, 64 * P) for L in lengths])
    inp = make_inputs(cfg, seed=31 + H)
    nb = inp.kv_cache.shape[0]
    poison = torch.full((4, 64, 1, 576), float("nan"), dtype=inp.kv_cache.dtype)
    kv = torch.cat([inp.kv_cache, poison])
    wide = torch.full((B, P + 4), nb, dtype=torch.int32)
    wide[:, P:] = torch.arange(nb, nb + 4, dtype=torch.int32)
    wide[:, :P] = inp.block_table[:, :P]
    say(f"length past the block table: H={H} s_q={s_q} splits={splits}")
    d = inp.to(gpu)
    kv_d = kv.to(gpu)
    table = wide.to(gpu)[:, :P]
    assert table.stride(0) == P + 4 and table.shape[1] == P
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    seqlens = torch.tensor(lengths, dtype=torch.int32, device=gpu)
    out, lse = mla_decode_with_kvcache(d.q, kv_d, table, seqlens, num_splits=splits,
                                       sm_scale=inp.sm_scale, causal=True, status=status)
    torch.cuda.synchronize()
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, True)
    assert_parity(out, lse, ref_o, ref_l, "past the table width")
    assert int(status.item()) == 1
    # the same batch within bounds leaves the status alone
    status.zero_()
    out2, lse2 = mla_decode_with_kvcache(d.q, kv_d, table, d.cache_seqlens, num_splits=splits,
                                         sm_scale=inp.sm_scale, causal=True, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert_parity(out2, lse2, ref_o, ref_l, "within the table width")


@pytest.mark.parametrize("H", [16, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_reference_fallback_pass(gpu, H, dtype):
    """Scores far above the first stage's row max force the exact two-pass redo of a segment.

    The rope dims of every token past the first 32 of a sequence are scaled by 100: the
    scaled scores then spread by ~30 natural-log units (far more than the reference margin of
    64 / 15 log2 units for bf16 / fp16).  Such softmaxes are dominated by single tokens, so
    out ~ one V row; the latent dims (V) are scaled by 1/4 to keep |out| < 2, where the bf16
    rounding of the output itself stays below 0.004 (at |out| >= 4 half a bf16 ulp alone is
    0.0156, beyond the 1e-2 bar for any bf16 output)."""
    lengths = [200, 64, 1000, 33]
    cfg = small_cfg(f"fallback_h{H}", len(lengths), 1, H, lengths, dtype)
    inp = make_inputs(cfg, seed=21)
    inp.kv_cache[..., :512] *= 0.25
    for b, L in enumerate(lengths):
        t = torch.arange(32, L)
        pages = inp.block_table[b, t // 64].long()
        inp.kv_cache[pages, t % 64, 0, 512:] *= 100
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, True)
    assert ref_l.max() - ref_l.min() > 20  # the scores really did spread
    for ns in (None, 1, 3):
        say(f"fallback H={H} dtype={dtype} num_splits={ns}")
        out, lse = run_paged(inp, gpu, ns)
        assert_parity(out, lse, ref_o, ref_l, f"fallback H={H} ns={ns}")


def _band_inputs(H, lengths, seed):
    """bf16 inputs whose every output lies in [2, 4): the latent dims (V) are drawn uniform in
    [2, 4), so each output row is a convex combination of values in that band.  Queries are
    scaled by 3 so each row's softmax mixes a few dozen keys unevenly."""
    cfg = small_cfg(f"band_h{H}", len(lengths), 1, H, lengths)
    inp = make_inputs(cfg, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    lat = 2 + 2 * torch.rand(inp.kv_cache.shape[:-1] + (512,), generator=g)
    inp.kv_cache[..., :512] = lat.to(torch.bfloat16)
    inp.q.mul_(3)
    return inp


@pytest.mark.parametrize("H", [16, 64, 128])
def test_multi_split_outputs_in_2_4(gpu, H):
    """Split partials must not add a second rounding: for bf16 outputs in [2, 4) half an ulp is
    2^-7 = 0.0078, and merging partials already rounded to bf16 reaches ~0.014 (see
    tests/test_oracle.py::test_bf16_partials_break_the_bar), past the 1e-2 bar."""
    inp = _band_inputs(H, [1024, 700, 2000, 4096], seed=31)
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, True)
    assert ref_o.min() >= 2 and ref_o.max() < 4
    for ns in (None, 2, 4, 8):
        say(f"band [2,4) H={H} num_splits={ns}")
        out, lse = run_paged(inp, gpu, ns)
        if ns is not None:
            _, splits = get_mla_metadata(inp.cache_seqlens.to(gpu), H, 1, forced_splits=ns)
            assert (splits[1:] - splits[:-1]).min().item() >= 2  # every sequence is split
        assert_parity(out, lse, ref_o, ref_l, f"band H={H} ns={ns}")


@pytest.mark.parametrize("H,dtype", [(16, torch.bfloat16), (16, torch.float16), (128, torch.bfloat16)])
def test_many_splits_per_sequence(gpu, H, dtype):
    """Sequences split 9 to 300 ways, against the oracle: the combine's general merge (rows of
    more than 8 splits, four rows per workgroup) and its dim-quarter form for long merges
    (16 or more parts per sequence: a register queue of 32 partial rows, surplus reads past the
    last split zeroed), with counts that leave a partial last round of the queue, and the plain
    merge past 256 splits.  Forced splits give min(splits, pages) non-empty page ranges, so
    every split here holds keys; splits without a visible key are covered by
    test_split_with_no_visible_key."""
    cfg = small_cfg(f"many_h{H}", 2, 1, H, [16384, 4001], dtype)
    inp = make_inputs(cfg, seed=40 + H)
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, True)
    for ns in (None, 9, 12, 40, 200, 256, 300):
        say(f"many splits H={H} dtype={dtype} num_splits={ns}")
        out, lse = run_paged(inp, gpu, ns)
        assert_parity(out, lse, ref_o, ref_l, f"many splits H={H} ns={ns}")


@pytest.mark.parametrize("B,L,ns", [(1, 64 * 7 + 1, 8), (1, 64 * 63 + 1, 64), (2, 64 * 11 + 1, 12)])
def test_split_with_no_visible_key(gpu, B, L, ns):
    """Causal s_q = 2 where the last split is one page holding only the last token: query 0
    sees no key of that split, so its partial has lse = -inf there, and the merge must give it
    weight 0.  Covers the few-splits merge (8 splits), the dim-quarter merge (64 splits, one
    sequence: 16 or more parts per sequence) and the general one (12 splits, two sequences)."""
    cfg = small_cfg(f"noviskey_{ns}", B, 2, 16, [L] * B)
    inp = make_inputs(cfg, seed=ns)
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, True)
    say(f"split without a visible key: L={L} num_splits={ns}")
    out, lse = run_paged(inp, gpu, ns)
    _, splits = get_mla_metadata(inp.cache_seqlens.to(gpu), 32, 1, forced_splits=ns)
    assert int(splits[1].item()) == ns  # one split per page at the end: the last holds one token
    assert_parity(out, lse, ref_o, ref_l, f"no visible key L={L} ns={ns}")


def _handmade_runner():
    """The library bound exactly as the reference binds its handmade kernel
    (handmade/mla_handmade.py:97-107): CDLL, argtypes [c_void_p] * 7 + [c_int], restype None."""
    import ctypes
    from mlc_decode_amd import _lib
    lib = ctypes.CDLL(_lib.library_path())
    fn = lib.mla_launch
    fn.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_int]
    fn.restype = None
    return fn


@pytest.mark.parametrize("sigma", [0.1, 1.0])
def test_mla_launch_reference_binding(gpu, sigma):
    """mla_launch(Q, Qpe, KV, Kpe, glse, partial, out, ns) on the reference's frozen shape
    (1 x 16 heads x 8192 tokens, fp16, caller-owned glse [1,16,ns+64] / partial [1,16,ns,576]
    scratch, handmade/mla_handmade.py:109-118) against the oracle."""
    fn = _handmade_runner()
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: (torch.randn(*s, generator=g) * sigma).to(torch.float16)  # noqa: E731
    q, qp, kv, kp = mk(1, 16, 512), mk(1, 16, 64), mk(1, 8192, 1, 512), mk(1, 8192, 1, 64)
    ref = R.decode_contiguous(q, qp, kv, kp)
    dq, dqp, dkv, dkp = (t.to(gpu) for t in (q, qp, kv, kp))
    for ns in (1, 3, 64, 128):
        say(f"mla_launch sigma={sigma} ns={ns}")
        glse = torch.zeros(1, 16, ns + 64, dtype=torch.float16, device=gpu)
        partial = torch.zeros(1, 16, ns, 576, dtype=torch.float16, device=gpu)
        out = torch.zeros(1, 16, 512, dtype=torch.float16, device=gpu)
        fn(dq.data_ptr(), dqp.data_ptr(), dkv.data_ptr(), dkp.data_ptr(), glse.data_ptr(),
           partial.data_ptr(), out.data_ptr(), ns)
        torch.cuda.synchronize()
        assert_parity(out, None, ref, None, f"mla_launch ns={ns}")
    # an invalid split count launches nothing
    out = torch.zeros(1, 16, 512, dtype=torch.float16, device=gpu)
    fn(dq.data_ptr(), dqp.data_ptr(), dkv.data_ptr(), dkp.data_ptr(), glse.data_ptr(),
       partial.data_ptr(), out.data_ptr(), 0)
    torch.cuda.synchronize()
    assert torch.all(out == 0)


def test_golden_fixtures_on_gpu(gpu):
    import numpy as np
    from test_oracle import GOLDEN, load_case
    z = np.load(GOLDEN)
    for name in sorted({k.split(".")[0] for k in z.files}):
        c = load_case(z, name)
        say(f"golden {name}")
        d = lambda t: t.to(gpu)  # noqa: E731
        out, lse = mla_decode_with_kvcache(d(c["q"]), d(c["kv"]), d(c["table"]), d(c["lengths"]),
                                           sm_scale=R.D_QK ** -0.5, causal=c["causal"])
        torch.cuda.synchronize()
        assert_parity(out, lse, c["out"], c["lse"], name)


def test_schedule_device_matches_host(gpu):
    rng = random.Random(5)
    cases = [
        [0, 1, 4096, 65, 16384, 128, 7000],
        [4096] * 64,
        # more sequences than the metadata kernel's threads: several per replay chunk
        [rng.choice([0, 1, 64, rng.randint(1, 9000)]) for _ in range(700)],
        [rng.randint(0, 3000) for _ in range(257)],   # two sequences per chunk, 129 chunks
        [5],
        [rng.randint(1, 200000) for _ in range(16384)],  # the largest batch: 256 walk windows
        [0] * 300,                                      # no pages: the serial pass
        [2**31 - 64] * 40,                              # 2^31 pages in total: the 64-bit serial pass
    ]
    for lengths in cases:
        seq = torch.tensor(lengths, dtype=torch.int32, device=gpu)
        for parts, fo, forced in ((256, -1, 0), (1024, -1, 0), (1, -1, 0), (7, 0, 0), (256, 5, 0),
                                  (0, -1, 3)):
            say(f"schedule B={len(lengths)} parts={parts} fo={fo} forced={forced}")
            s_d, n_d = get_mla_metadata(seq, 16, 1, num_parts=parts or None, fixed_overhead=fo,
                                        forced_splits=forced)
            s_h, n_h = get_mla_metadata_host(lengths, parts, fo, forced)
            torch.cuda.synchronize()
            assert torch.equal(s_d.cpu(), s_h) and torch.equal(n_d.cpu(), n_h)


def test_flash_mla_call_shape(gpu):
    cfg = small_cfg("flash", 2, 1, 16, [100, 2000])
    inp = make_inputs(cfg, seed=11).to(gpu)
    say("flash_mla_with_kvcache")
    meta, splits = get_mla_metadata(inp.cache_seqlens, 16, 1)
    out, lse = flash_mla_with_kvcache(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens, 512,
                                      meta, splits, causal=True)
    cpu = make_inputs(cfg, seed=11)
    ref_o, ref_l = R.decode_paged(cpu.q, cpu.kv_cache, cpu.block_table, cpu.cache_seqlens,
                                  cpu.sm_scale, True)
    assert_parity(out, lse, ref_o, ref_l, "flash_mla")


@pytest.mark.parametrize("H,s_q", [(16, 1), (64, 1), (128, 1), (128, 2)])
def test_split_latent_rope_views(gpu, H, s_q):
    """Latent and rope halves in separate allocations: the kernels' general form, where the rope
    rows are looked up through their own page base (the benchmark caches are one [.., 576]
    tensor, whose rope half the 64- and 128-row kernels read at the latent row + 1024 bytes)."""
    cfg = small_cfg(f"views_h{H}_s{s_q}", 2, s_q, H, [70, 130])
    cpu = make_inputs(cfg, seed=12)
    inp = cpu.to(gpu)
    latent = inp.kv_cache[..., :512].contiguous()
    rope = inp.kv_cache[..., 512:].contiguous()
    say(f"separate latent / rope tensors: H={H} s_q={s_q}")
    out, lse = mla_decode_with_kvcache(inp.q, (latent, rope), inp.block_table, inp.cache_seqlens)
    ref_o, ref_l = R.decode_paged(cpu.q, cpu.kv_cache, cpu.block_table, cpu.cache_seqlens,
                                  cpu.sm_scale, True)
    assert_parity(out, lse, ref_o, ref_l, "views")


def test_merge_partials(gpu):
    g = torch.Generator().manual_seed(13)
    splits = torch.tensor([0, 3, 4, 9], dtype=torch.int32)
    rows = 20
    part_o = torch.randn(9, rows, 512, generator=g)
    part_l2 = torch.randn(9, rows, generator=g) * 4
    part_l2[1, 3] = -math.inf           # one empty split
    part_l2[3, :] = -math.inf           # a sequence whose only split is empty
    say("merge_partials")
    out, lse = merge_partials(part_o.to(gpu), part_l2.to(gpu), splits.to(gpu), torch.bfloat16)
    torch.cuda.synchronize()
    ln = part_l2 * math.log(2)
    for b in range(3):
        a, e = int(splits[b]), int(splits[b + 1])
        ro, rl = R.combine(part_o[a:e], ln[a:e])
        if e - a == 1 and torch.isinf(rl).all():
            ro = part_o[a] * 0
        assert_parity(out[b].unsqueeze(0), lse[b].unsqueeze(0), ro.unsqueeze(0), rl.unsqueeze(0),
                      f"merge b={b}")


# ---------------------------------------------------------------- reference call shapes
@pytest.mark.parametrize("kv_ctx", [7, 33, 2048, 3000, 3008, 4095, 4096])
def test_reference_contiguous_layout(gpu, kv_ctx, monkeypatch):
    import baseline_mla
    import mla_decode
    monkeypatch.setattr(mla_decode, "_AUTOTUNE_ENABLED", False)
    g = torch.Generator().manual_seed(kv_ctx)
    b, h = 1, 16
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.1).to(torch.float16)  # noqa: E731
    q, q_pe, kv, k_pe = mk(b, h, 512), mk(b, h, 64), mk(b, kv_ctx, 1, 512), mk(b, kv_ctx, 1, 64)
    ref = R.decode_contiguous(q, q_pe, kv, k_pe)
    args = [t.to(gpu) for t in (q, q_pe, kv, k_pe)]
    for name, kern in (("mla_decode", mla_decode._get_kernel(b, h, 1, kv_ctx, 512, 64)),
                       ("baseline_mla", baseline_mla._get_kernel(b, h, 1, kv_ctx, 512, 64)),
                       ("explicit ns=5", mla_decode.build_kernel_from_config(
                           b, h, 1, kv_ctx, 512, 64, {"num_split": 5, "block_N": 32, "block_H": 16}))):
        say(f"contiguous {name} kv_ctx={kv_ctx}")
        out = torch.empty_like(args[0])
        kern(*args, out)
        torch.cuda.synchronize()
        assert_parity(out, None, ref, None, f"{name} ctx={kv_ctx}")
        # repeat calls reuse the prepared arguments: same tensors into a second output, a
        # returned output, then new input tensors (a changed key), each checked
        out2 = torch.empty_like(args[0])
        kern(*args, out2)
        out3 = kern(*args)
        fresh = [t.clone() for t in args]
        out4 = torch.empty_like(args[0])
        kern(*fresh, out4)
        torch.cuda.synchronize()
        assert torch.equal(out2, out) and torch.equal(out3, out) and torch.equal(out4, out)
    assert_parity(baseline_mla.ref_program(*args), None, ref, None, "ref_program")


@pytest.mark.parametrize("kv_ctx", [100, 4096])
@pytest.mark.parametrize("h", [64, 128])
def test_reference_factories_and_run_kernel(gpu, kv_ctx, h, monkeypatch):
    """The explicit-config factories (mla_decode.py:33-39, :263; called by
    scripts/bench_mla_heads.py:130-136 with TileLang knobs) and run_kernel (:715-717)."""
    import mla_decode
    monkeypatch.setattr(mla_decode, "_AUTOTUNE_ENABLED", False)
    g = torch.Generator().manual_seed(kv_ctx + h)
    b = 2
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.1).to(torch.float16)  # noqa: E731
    q, q_pe, kv, k_pe = mk(b, h, 512), mk(b, h, 64), mk(b, kv_ctx, 1, 512), mk(b, kv_ctx, 1, 64)
    ref = R.decode_contiguous(q, q_pe, kv, k_pe)
    args = [t.to(gpu) for t in (q, q_pe, kv, k_pe)]
    scale = 576 ** -0.5
    for name, factory in (("flashattn_shared_q", mla_decode.flashattn_shared_q),
                          ("flashattn_frag_q", mla_decode.flashattn_frag_q)):
        for num_split in (1, 4):
            kern = factory(b, h, 1, kv_ctx, 512, 64, 64, 64, num_split, 2, 8, scale, threads=256)
            say(f"{name} kv_ctx={kv_ctx} num_split={num_split}")
            out = torch.empty_like(args[0])
            assert kern(*args, out) is None
            torch.cuda.synchronize()
            assert_parity(out, None, ref, None, f"{name} ns={num_split}")
    say(f"run_kernel kv_ctx={kv_ctx}")
    out = torch.empty_like(args[0])
    mla_decode.run_kernel(*args, out, b, h, 1, kv_ctx, 512, 64)
    torch.cuda.synchronize()
    assert_parity(out, None, ref, None, "run_kernel")


def test_reference_autotune_path(gpu):
    import mla_decode
    say("mla_decode._get_kernel autotune b=2 h=64 ctx=1500")
    k = mla_decode._get_kernel(2, 64, 1, 1500, 512, 64)
    g = torch.Generator().manual_seed(3)
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.1).to(torch.float16)  # noqa: E731
    q, q_pe, kv, k_pe = mk(2, 64, 512), mk(2, 64, 64), mk(2, 1500, 1, 512), mk(2, 1500, 1, 64)
    out = k(*[t.to(gpu) for t in (q, q_pe, kv, k_pe)])
    torch.cuda.synchronize()
    assert_parity(out, None, R.decode_contiguous(q, q_pe, kv, k_pe), None, "autotuned")


# ---------------------------------------------------------------- benchmark configs
@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_benchmark_config(gpu, name):
    """Every sequence of every benchmark config at full size against the oracle (the fp32
    oracle takes well under a second per config on the host cores)."""
    cfg = CONFIGS[name]
    inp = make_inputs(cfg, seed=0)
    say(f"config {name} B={cfg.batch} H={cfg.heads} s_q={cfg.s_q} num_splits={cfg.num_splits}")
    out, lse = run_paged(inp, gpu, cfg.num_splits)
    if cfg.num_splits:
        _, splits = get_mla_metadata(inp.cache_seqlens.to(gpu), cfg.s_q * cfg.heads, 1,
                                     forced_splits=cfg.num_splits)
        per_seq = (splits[1:] - splits[:-1]).cpu()
        pages = (inp.cache_seqlens + 63) // 64
        assert torch.equal(per_seq, torch.minimum(pages, torch.full_like(pages, cfg.num_splits)).clamp(min=1))
    assert torch.isfinite(out.float()).all()
    assert torch.isfinite(lse).all() or cfg.s_q > 1
    ref_o, ref_l = R.decode_paged(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                  inp.sm_scale, inp.causal)
    assert_parity(out, lse, ref_o, ref_l, name)


# ---------------------------------------------------------------- paged KV-cache append
def _append_inputs(seed, lens, n_new, P, dtype):
    g = torch.Generator().manual_seed(seed)
    lens = torch.tensor(lens, dtype=torch.int32)
    B = len(lens)
    N = B * P + 7
    bt = torch.randperm(N, generator=g)[: B * P].to(torch.int32).view(B, P)
    cache = torch.randn(N, 64, 1, 576, generator=g).to(dtype)
    new = torch.randn(B, n_new, 576, generator=g).to(dtype)
    return cache, bt, lens, new


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n_new", [1, 2, 3])
def test_kv_append_matches_oracle(gpu, dtype, n_new):
    """Bit-exact against the oracle, rows crossing page boundaries, one tensor or two views."""
    cache, bt, lens, new = _append_inputs(40 + n_new, [0, 1, 62, 63, 64, 127, 200, 255], n_new, 5, dtype)
    want_cache, want_lens, skipped = R.append_paged(cache, bt, lens, new)
    assert skipped == []
    for views in (False, True):
        say(f"kv_append dtype={dtype} n_new={n_new} views={views}")
        c = cache.to(gpu)
        kvc = (c[..., :512], c[..., 512:]) if views else c
        ln = lens.to(gpu)
        st = torch.zeros(1, dtype=torch.int32, device=gpu)
        kv_append(new.to(gpu), kvc, bt.to(gpu), ln, status=st)
        torch.cuda.synchronize()
        assert torch.equal(c.cpu(), want_cache)
        assert torch.equal(ln.cpu(), want_lens)
        assert st.item() == 0


def test_kv_append_skips_unassigned_pages(gpu):
    cache, bt, lens, new = _append_inputs(7, [10, 4 * 64 - 1, 64, 63, 5], 2, 4, torch.bfloat16)
    bt[3, 1] = cache.shape[0]  # sequence 3 crosses into a page id past the cache
    want_cache, want_lens, skipped = R.append_paged(cache, bt, lens, new)
    assert skipped == [1, 3]
    say("kv_append with unassigned pages")
    c, ln = cache.to(gpu), lens.to(gpu)
    st = torch.zeros(1, dtype=torch.int32, device=gpu)
    kv_append(new.to(gpu), c, bt.to(gpu), ln, status=st)
    torch.cuda.synchronize()
    assert st.item() == 1
    assert torch.equal(c.cpu(), want_cache) and torch.equal(ln.cpu(), want_lens)


@pytest.mark.parametrize("H", [16, 128])
def test_kv_append_then_decode(gpu, H):
    """Decode over the appended cache matches the oracle decode of the extended sequences."""
    cache, bt, lens, new = _append_inputs(11, [1, 63, 64, 300, 0], 1, 6, torch.bfloat16)
    want_cache, want_lens, _ = R.append_paged(cache, bt, lens, new)
    g = torch.Generator().manual_seed(12)
    q = torch.randn(len(lens), 1, H, 576, generator=g).to(torch.bfloat16)
    say(f"kv_append then decode H={H}")
    c, ln, btg = cache.to(gpu), lens.to(gpu), bt.to(gpu)
    kv_append(new.to(gpu), c, btg, ln)
    out, lse = mla_decode_with_kvcache(q.to(gpu), c, btg, ln, sm_scale=576 ** -0.5, causal=True)
    torch.cuda.synchronize()
    ref_o, ref_l = R.decode_paged(q, want_cache, bt, want_lens, 576 ** -0.5, True)
    assert_parity(out, lse, ref_o, ref_l, f"append+decode H={H}")
