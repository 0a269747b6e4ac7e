"""Pins the CPU oracle (oracle/mla_ref.py) before it is trusted as the GPU checker.

Each check is one a plausible oracle mistake fails: a library routine computed
independently (torch SDPA / logsumexp in float64, via the committed fixtures), closed
forms (L = 1, q = 0, identical keys), invariances (page permutation, splitting + merge,
query scaling), the causal rule (s_q = 2 rows vs s_q = 1 decodes) and brute-force integer
checks of the split rule and the schedules.
"""
import math
import os
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mla_ref as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "mla_cases.npz")


def load_case(z, name):
    s_q, H, dt, causal = (int(x) for x in z[f"{name}.meta"])
    dtype = torch.bfloat16 if dt == 0 else torch.float16
    q = torch.from_numpy(z[f"{name}.q"]).view(dtype)
    kv = torch.from_numpy(z[f"{name}.kv"]).view(dtype)
    return dict(q=q, kv=kv, table=torch.from_numpy(z[f"{name}.table"]),
                lengths=torch.from_numpy(z[f"{name}.lengths"]), causal=bool(causal),
                out=torch.from_numpy(z[f"{name}.out"]), lse=torch.from_numpy(z[f"{name}.lse"]))


def rand_paged(B, s_q, H, lengths, dtype=torch.float32, seed=0, sigma=1.0):
    g = torch.Generator().manual_seed(seed)
    pages = [R.pages_of(L) for L in lengths]
    total = max(sum(pages), 1)
    perm = torch.randperm(total, generator=g)
    table = torch.zeros(B, max(max(pages), 1), dtype=torch.int32)
    off = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = (torch.randn(B, s_q, H, R.D_QK, generator=g) * sigma).to(dtype)
    kv = (torch.randn(total, R.PAGE, 1, R.D_QK, generator=g) * sigma).to(dtype)
    return q, kv, table, torch.tensor(lengths, dtype=torch.int32)


SCALE = R.D_QK ** -0.5


def test_golden_fixtures():
    z = np.load(GOLDEN)
    names = sorted({k.split(".")[0] for k in z.files})
    assert len(names) >= 6
    for name in names:
        c = load_case(z, name)
        out, lse = R.decode_paged(c["q"], c["kv"], c["table"], c["lengths"], SCALE, c["causal"])
        assert torch.allclose(out, c["out"], atol=2e-5, rtol=1e-4), name
        fin = torch.isfinite(c["lse"])
        assert torch.equal(fin, torch.isfinite(lse)), name
        assert torch.allclose(lse[fin], c["lse"][fin], atol=2e-5, rtol=1e-5), name
        assert torch.all(out[~fin.permute(0, 2, 1)] == 0), name


def test_sdpa_library_float64():
    q, kv, table, lens = rand_paged(3, 1, 16, [1, 70, 190], torch.float64, seed=3)
    out, _ = R.decode_paged(q, kv, table, lens, SCALE, causal=True, dtype=torch.float64)
    for b in range(3):
        k = R.gather(kv[:, :, 0], table[b], int(lens[b]))
        ref = F.scaled_dot_product_attention(q[b].transpose(0, 1).unsqueeze(0),
                                             k.expand(16, -1, -1).unsqueeze(0),
                                             k[:, :512].expand(16, -1, -1).unsqueeze(0), scale=SCALE)
        assert torch.allclose(out[b, 0], ref[0, :, 0], atol=1e-12)


def test_length_one_closed_form():
    q, kv, table, lens = rand_paged(2, 1, 16, [1, 1], torch.float64, seed=4)
    out, lse = R.decode_paged(q, kv, table, lens, SCALE, dtype=torch.float64)
    for b in range(2):
        k0 = kv[table[b, 0].long(), 0, 0]
        assert torch.allclose(out[b, 0], k0[:512].expand(16, -1), atol=1e-12)
        assert torch.allclose(lse[b, :, 0], (q[b, 0] @ k0) * SCALE, atol=1e-12)


def test_zero_query_is_uniform():
    q, kv, table, lens = rand_paged(2, 1, 16, [37, 300], torch.float64, seed=5)
    q.zero_()
    out, lse = R.decode_paged(q, kv, table, lens, SCALE, dtype=torch.float64)
    for b, L in enumerate([37, 300]):
        k = R.gather(kv[:, :, 0], table[b], L)
        assert torch.allclose(out[b, 0], k[:, :512].mean(0).expand(16, -1), atol=1e-12)
        assert torch.allclose(lse[b, :, 0], torch.full((16,), math.log(L), dtype=torch.float64))


def test_identical_keys():
    q, kv, table, lens = rand_paged(1, 1, 16, [150], torch.float64, seed=6)
    kv[:] = kv[0, 0]
    out, lse = R.decode_paged(q, kv, table, lens, SCALE, dtype=torch.float64)
    k = kv[0, 0, 0]
    assert torch.allclose(out[0, 0], k[:512].expand(16, -1), atol=1e-12)
    assert torch.allclose(lse[0, :, 0], q[0, 0] @ k * SCALE + math.log(150), atol=1e-12)


def test_page_permutation_invariance():
    q, kv, table, lens = rand_paged(2, 1, 16, [130, 250], seed=7)
    out, lse = R.decode_paged(q, kv, table, lens, SCALE)
    perm = torch.randperm(kv.shape[0], generator=torch.Generator().manual_seed(1))
    inv = torch.argsort(perm)
    out2, lse2 = R.decode_paged(q, kv[perm], inv[table.long()].to(torch.int32), lens, SCALE)
    assert torch.allclose(out, out2, atol=1e-6) and torch.allclose(lse, lse2, atol=1e-6)


def test_split_and_merge():
    # two halves of the key set as two sequences, merged, equal the whole
    q, kv, table, lens = rand_paged(1, 1, 16, [256], torch.float64, seed=8)
    whole_o, whole_l = R.decode_paged(q, kv, table, lens, SCALE, dtype=torch.float64)
    halves = torch.stack([table[0, :2], table[0, 2:4]])
    o2, l2 = R.decode_paged(q.expand(2, -1, -1, -1), kv, halves, torch.tensor([128, 128]), SCALE,
                            dtype=torch.float64)
    mo, ml = R.combine(o2[:, 0], l2[:, :, 0])
    assert torch.allclose(mo, whole_o[0, 0], atol=1e-12)
    assert torch.allclose(ml, whole_l[0, :, 0], atol=1e-12)


def test_query_scaling():
    q, kv, table, lens = rand_paged(1, 1, 16, [99], torch.float64, seed=9)
    o1, l1 = R.decode_paged(q, kv, table, lens, SCALE, dtype=torch.float64)
    o2, l2 = R.decode_paged(q * 3.0, kv, table, lens, SCALE / 3.0, dtype=torch.float64)
    assert torch.allclose(o1, o2, atol=1e-12) and torch.allclose(l1, l2, atol=1e-12)


def test_causal_rows_match_single_query_decodes():
    q, kv, table, lens = rand_paged(2, 2, 16, [1, 77], torch.float64, seed=10)
    out, lse = R.decode_paged(q, kv, table, lens, SCALE, causal=True, dtype=torch.float64)
    for i, shift in ((1, 0), (0, 1)):
        lens_i = lens - shift
        o1, l1 = R.decode_paged(q[:, i:i + 1], kv, table, lens_i, SCALE, dtype=torch.float64)
        assert torch.allclose(out[:, i], o1[:, 0], atol=1e-12)
        assert torch.equal(torch.isinf(lse[:, :, i]), torch.isinf(l1[:, :, 0]))
    # L = 1 with s_q = 2: query 0 sees nothing
    assert torch.all(out[0, 0] == 0) and torch.all(torch.isinf(lse[0, :, 0]))


def test_contiguous_equals_identity_paged():
    g = torch.Generator().manual_seed(11)
    B, H, L = 2, 16, 128
    q, q_pe = torch.randn(B, H, 512, generator=g), torch.randn(B, H, 64, generator=g)
    kv, k_pe = torch.randn(B, L, 1, 512, generator=g), torch.randn(B, L, 1, 64, generator=g)
    ref = R.decode_contiguous(q, q_pe, kv, k_pe)
    cache = torch.cat([kv, k_pe], -1).reshape(B * L // 64, 64, 1, 576)
    table = torch.arange(B * L // 64, dtype=torch.int32).reshape(B, -1)
    out, _ = R.decode_paged(torch.cat([q, q_pe], -1).unsqueeze(1), cache, table,
                            torch.full((B,), L, dtype=torch.int32), SCALE)
    assert torch.allclose(out[:, 0], ref, atol=1e-5)


def test_split_plan_bruteforce():
    for L in list(range(1, 300, 7)) + [2048, 3000, 4095, 4096, 8192, 16384, 65536]:
        for block_n in (16, 32, 64):
            nb = -(-L // block_n)
            for ns_req in (1, 2, 3, 7, 64, 104, 208, 312, 1024):
                ns, bpc, extra = R.split_plan(L, ns_req, block_n, False)
                assert extra == 0 and ns * bpc >= nb and (ns - 1) * bpc < nb
                ns, bpc, extra = R.split_plan(L, ns_req, block_n, True)
                assert ns == max(1, min(ns_req, nb)) and ns * bpc + extra == nb and extra < ns
    # the reference's recorded best configs are coverable splits
    assert R.split_plan(16384, 104, 32, True) == (104, 4, 96)
    assert R.split_plan(8192, 312, 32, False)[0] == 256


def _check_schedule(lengths, recs, prefix, num_parts):
    segs = R.segments(recs, lengths)
    covered = {}
    for p, b, pb, pe, sp in segs:
        for pg in range(pb, pe):
            assert (b, pg) not in covered
            covered[(b, pg)] = p
        covered.setdefault(("seq", b), []).append(sp)
    for b, L in enumerate(lengths):
        for pg in range(R.pages_of(L)):
            assert (b, pg) in covered
        splits = covered[("seq", b)]
        assert sorted(splits) == list(range(len(splits)))
        assert prefix[b + 1] - prefix[b] == len(splits)


@pytest.mark.parametrize("seed", range(6))
def test_balanced_schedule_bruteforce(seed):
    rng = random.Random(seed)
    B = rng.choice([1, 3, 17, 64, 132])
    lengths = [rng.choice([0, 1, 63, 64, 65, rng.randint(1, 20000)]) for _ in range(B)]
    for parts in (1, 7, 64, 256):
        for fo in (0, 2, 5):
            recs, prefix = R.schedule_balanced(lengths, parts, fo)
            assert len(recs) == parts
            _check_schedule(lengths, recs, prefix, parts)
            total = sum(R.pages_of(L) + fo for L in lengths)
            payload = -(-total // parts) + fo
            for p, b, pb, pe, sp in R.segments(recs, lengths):
                if p < parts - 1:
                    assert pe - pb <= payload


@pytest.mark.parametrize("seed", range(6))
def test_min_payload_schedule_bruteforce(seed):
    """The default schedule: a valid cover, every part within the chosen payload, and no
    smaller payload fits; the explicit-payload loop agrees with the reference loop where
    both apply."""
    rng = random.Random(50 + seed)
    B = rng.choice([1, 3, 17, 64, 132])
    lengths = [rng.choice([0, 1, 63, 64, 65, rng.randint(1, 20000)]) for _ in range(B)]
    for parts in (1, 7, 64, 256, 1024):
        for fo in (0, 1, 2, 5):
            recs, prefix, payload = R.schedule_min_payload(lengths, parts, fo)
            assert len(recs) == parts
            _check_schedule(lengths, recs, prefix, parts)
            total = sum(R.pages_of(L) + fo for L in lengths)
            lo = -(-total // parts)
            assert lo <= payload <= lo + fo
            if payload > lo:
                assert R.pack_greedy(lengths, parts, payload - 1, fo) is None
            cost = [0] * parts
            for p, b, pb, pe, sp in R.segments(recs, lengths):
                cost[p] += pe - pb + fo
            assert max(cost) <= payload
            # at the reference payload the explicit loop is the reference loop
            bal = R.schedule_balanced(lengths, parts, fo)
            assert R.pack_greedy(lengths, parts, lo + fo, fo) == bal


def test_min_payload_uniform_closed_form():
    """Uniform lengths with parts = k * batch: every part is exactly pages / k pages of one
    sequence (the shape of the B=64, L=4096 decode on 256 parts)."""
    for B, L, k, fo in ((64, 4096, 4, 2), (64, 4096, 4, 5), (32, 16384, 4, 2), (8, 1024, 2, 0)):
        recs, prefix, payload = R.schedule_min_payload([L] * B, B * k, fo)
        per = R.pages_of(L) // k
        assert payload == per + fo
        assert prefix == [k * b for b in range(B + 1)]
        assert recs == [(i // k, (i % k) * per, i // k, (i % k + 1) * per, i % k)
                        if (i % k) < k - 1 else (i // k, (i % k) * per, i // k + 1, 0, i % k)
                        for i in range(B * k)]


def test_forced_schedule_bruteforce():
    lengths = [0, 1, 64, 65, 1000, 4096]
    for forced in (1, 2, 3, 8):
        recs, prefix = R.schedule_forced(lengths, forced)
        assert len(recs) == len(lengths) * forced
        _check_schedule(lengths, recs, prefix, len(recs))
        for b, L in enumerate(lengths):
            assert prefix[b + 1] - prefix[b] == max(1, min(forced, R.pages_of(L)))


def test_oracle_mistakes_are_caught():
    """Planted mistakes in the oracle (dropping the rope dims, a wrong scale, a reversed page
    walk) each fail the fixture check."""
    z = np.load(GOLDEN)
    c = load_case(z, "h16_tails")
    q = c["q"].clone()
    q[..., 512:] = 0  # what an oracle that forgot q_rope . k_rope would compute
    out, _ = R.decode_paged(q, c["kv"], c["table"], c["lengths"], SCALE, c["causal"])
    assert not torch.allclose(out, c["out"], atol=2e-5, rtol=1e-4)
    # a wrong softmax scale (the 512-d latent width instead of 576)
    out, lse = R.decode_paged(c["q"], c["kv"], c["table"], c["lengths"], 512 ** -0.5, c["causal"])
    assert not torch.allclose(out, c["out"], atol=2e-5, rtol=1e-4)
    # a transposed page walk: the pages of each sequence visited in reverse order
    table = c["table"].clone()
    for b, L in enumerate(c["lengths"].tolist()):
        n = R.pages_of(L)
        if n > 1:
            table[b, :n] = table[b, :n].flip(0)
    out, _ = R.decode_paged(c["q"], c["kv"], table, c["lengths"], SCALE, c["causal"])
    assert not torch.allclose(out, c["out"], atol=2e-5, rtol=1e-4)


def _append_case(seed, B=6, n=2, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    lens = torch.tensor([0, 1, 62, 63, 64, 130][:B], dtype=torch.int32)
    P = 4
    N = B * P + 3
    perm = torch.randperm(N, generator=g)[: B * P].to(torch.int32).view(B, P)
    cache = torch.randn(N, R.PAGE, 1, R.D_QK, generator=g).to(dtype)
    new = torch.randn(B, n, R.D_QK, generator=g).to(dtype)
    return cache, perm, lens, new


def test_append_oracle_against_gather():
    """Appending then gathering a sequence gives its old tokens followed by the new ones, and
    no other cache row changes."""
    cache, bt, lens, new = _append_case(0)
    out, lens2, skipped = R.append_paged(cache, bt, lens, new)
    assert skipped == []
    assert torch.equal(lens2, lens + new.shape[1])
    written = torch.zeros(cache.shape[:2], dtype=torch.bool)
    for b in range(len(lens)):
        L, L2 = int(lens[b]), int(lens2[b])
        got = R.gather(out[:, :, 0, :], bt[b], L2)
        want = torch.cat([R.gather(cache[:, :, 0, :], bt[b], L), new[b]])
        assert torch.equal(got, want)
        for pos in range(L, L2):
            written[int(bt[b, pos // R.PAGE]), pos % R.PAGE] = True
    assert torch.equal(out[~written], cache[~written])


def test_append_oracle_then_decode():
    """Decoding the appended paged cache equals the contiguous closed form over the
    concatenated tokens (the decode path consumes exactly what the append wrote)."""
    cache, bt, lens, new = _append_case(1, n=1, dtype=torch.float32)
    out, lens2, _ = R.append_paged(cache, bt, lens, new)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(len(lens), 1, 16, R.D_QK, generator=g)
    o_p, l_p = R.decode_paged(q, out, bt, lens2, R.D_QK ** -0.5, True)
    for b in range(len(lens)):
        kv = torch.cat([R.gather(cache[:, :, 0, :], bt[b], int(lens[b])), new[b]])
        o_c = R.decode_contiguous(q[b:b + 1, 0, :, :512], q[b:b + 1, 0, :, 512:],
                                  kv[None, :, None, :512], kv[None, :, None, 512:])
        assert torch.allclose(o_p[b, 0], o_c[0], atol=1e-5, rtol=1e-5)


def test_append_oracle_skips_unassigned_pages():
    cache, bt, lens, new = _append_case(2, n=2)
    bt = bt.clone()
    lens = lens.clone()
    lens[1] = 4 * R.PAGE - 1          # second token would need page slot 4 of a 4-slot table
    bt[3, 1] = cache.shape[0]         # a page id past the cache, used by sequence 3 (63, 64)
    out, lens2, skipped = R.append_paged(cache, bt, lens, new)
    assert skipped == [1, 3]
    assert lens2[1] == lens[1] and lens2[3] == lens[3]
    assert lens2[0] == lens[0] + 2


def test_sparse_oracle_equals_paged_through_dense_indices():
    torch.manual_seed(3)
    B, H, nb = 3, 16, 12
    kv = torch.randn(nb, 64, 1, 576)
    table = torch.randperm(nb).reshape(B, 4).to(torch.int32)
    lens = torch.tensor([1, 100, 256], dtype=torch.int32)
    q = torch.randn(B, 1, H, 576)
    ref_o, ref_l = R.decode_paged(q, kv, table, lens, 0.05, True)
    idx = R.dense_indices(table, lens, 300)
    o, l = R.decode_sparse(q, kv, idx, 0.05)
    assert torch.allclose(o, ref_o, atol=1e-5) and torch.allclose(l, ref_l, atol=1e-5)


def test_sparse_oracle_permutation_and_empty():
    torch.manual_seed(4)
    kv = torch.randn(4, 64, 1, 576)
    q = torch.randn(2, 1, 8, 576)
    idx = torch.tensor([[5, 70, 200, -1, 3], [-1, -1, 999999, -7, -1]], dtype=torch.int32)
    o, l = R.decode_sparse(q, kv, idx, 0.1)
    perm = idx[:, torch.tensor([4, 2, 0, 3, 1])]
    o2, l2 = R.decode_sparse(q, kv, perm, 0.1)
    assert torch.allclose(o, o2, atol=1e-6) and torch.allclose(l, l2, atol=1e-6)
    assert torch.all(o[1] == 0) and torch.all(l[1] == float("-inf"))   # no valid key
    # one key only: out is that key's latent, lse its score
    one = torch.tensor([[70], [70]], dtype=torch.int32)
    o3, l3 = R.decode_sparse(q, kv, one, 0.1)
    k = kv.reshape(-1, 576)[70]
    assert torch.allclose(o3[:, 0], k[:512].expand(2, 8, 512), atol=1e-6)
    assert torch.allclose(l3[:, :, 0], (q[:, 0] @ k) * 0.1, atol=1e-5)


def test_check_cli_reference_equals_oracle():
    # the check CLI's float32 reference (python -m mlc_decode_amd.check) computes the same
    # decode as the oracle, including grouped KV heads
    from mlc_decode_amd.check import torch_ref
    g = torch.Generator().manual_seed(4)
    for b, h, hk, ctx in ((1, 16, 1, 33), (2, 8, 2, 100)):
        q = torch.randn(b, h, 512, generator=g) * 0.1
        q_pe = torch.randn(b, h, 64, generator=g) * 0.1
        kv = torch.randn(b, ctx, hk, 512, generator=g) * 0.1
        k_pe = torch.randn(b, ctx, hk, 64, generator=g) * 0.1
        got = torch_ref(q, q_pe, kv, k_pe, b, h, hk, ctx, 512, 64)
        want = R.decode_contiguous(q, q_pe, kv, k_pe)
        assert torch.allclose(got, want, atol=1e-6, rtol=1e-5)


def _scaled_f16(po):
    """Split partials as the decode workspace holds them: fp16 times 2^e per 128-dim chunk of a
    row, e = 15 - E for chunk amax = m 2^E, m in [0.5, 1) (the chunk lands in [2^14, 2^15)),
    then multiplied back by 2^-e as the combine does."""
    out = po.clone()
    for c in range(4):
        ch = po[..., 128 * c:128 * (c + 1)]
        amax = ch.abs().amax(-1, keepdim=True)
        _, E = torch.frexp(amax)
        e = (15 - E).clamp(max=127).to(po.dtype)
        out[..., 128 * c:128 * (c + 1)] = (ch * torch.exp2(e)).to(torch.float16).to(po.dtype) * torch.exp2(-e)
    return out


def test_bf16_partials_break_the_bar():
    """Why the decode does not keep split partials in bf16.  Outputs in [2, 4) (latent dims
    drawn in that band) merged from 4 splits: with fp32 partials the error against the fp32
    oracle is the output's own bf16 rounding (<= 2^-7 = 0.0078); with partials rounded to bf16
    before the merge (the reference's partial format, mla_decode.py:73-74) it passes 1e-2; with
    the decode's scaled fp16 partials (2^-11 of each 128-dim chunk's amax, here <= 2^-10) it
    stays within 2^-7 + 2^-10."""
    g = torch.Generator().manual_seed(3)
    H, L, S = 16, 1024, 4
    q = (torch.randn(H, 576, generator=g) * 3).to(torch.bfloat16).double()
    k = torch.empty(L, 576, dtype=torch.float64)
    k[:, :512] = (2 + 2 * torch.rand(L, 512, generator=g, dtype=torch.float64)).to(torch.bfloat16).double()
    k[:, 512:] = torch.randn(L, 64, generator=g, dtype=torch.float64).to(torch.bfloat16).double()
    s = (q @ k.T) * 576 ** -0.5
    ref = torch.softmax(s, -1) @ k[:, :512]
    assert ref.min() >= 2 and ref.max() < 4
    parts, lses = [], []
    for c in range(S):  # each split's softmax-normalised output and natural-log lse
        sl = slice(c * L // S, (c + 1) * L // S)
        parts.append(torch.softmax(s[:, sl], -1) @ k[sl, :512])
        lses.append(torch.logsumexp(s[:, sl], -1))
    part_o, part_l = torch.stack(parts), torch.stack(lses)
    errs = {}
    for name, po in (("fp32", part_o.float()), ("bf16", part_o.to(torch.bfloat16).float()),
                     ("f16s", _scaled_f16(part_o.float()))):
        out, lse = R.combine(po, part_l.float())
        assert (lse.double() - torch.logsumexp(s, -1)).abs().max() < 1e-4
        errs[name] = (out.to(torch.bfloat16).double() - ref).abs().max().item()
    assert errs["fp32"] <= 2 ** -7 + 1e-6
    assert errs["bf16"] > 1e-2
    assert errs["f16s"] <= 2 ** -7 + 2 ** -10 + 1e-6 < 1e-2


def test_scaled_f16_partials_error_bound():
    """The scaled fp16 partial format on chunks of very different magnitudes, signs, zeros and
    extreme exponents: every value comes back within 2^-11 of its chunk's amax."""
    g = torch.Generator().manual_seed(4)
    po = torch.randn(3, 5, 512, generator=g, dtype=torch.float64)
    po[0, 0, :128] *= 1e-30          # tiny chunk
    po[0, 1, 128:256] *= 3e4         # large chunk
    po[1, 2, 256:384] = 0.0          # all-zero chunk
    po[2, 3, 384:] = -7.5            # constant negative chunk
    po[2, 4, :] *= 2.0 ** -100
    back = _scaled_f16(po.float()).double()
    for c in range(4):
        ch = po[..., 128 * c:128 * (c + 1)].float().double()
        amax = ch.abs().amax(-1, keepdim=True)
        err = (back[..., 128 * c:128 * (c + 1)] - ch).abs()
        assert torch.all(err <= amax * 2.0 ** -11)
