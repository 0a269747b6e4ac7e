"""C-ABI checks that need no GPU: the library loads, exports every symbol the header
declares, its host-side schedule and split rule agree with the oracle, and bad arguments
come back as nonzero statuses with messages (validation runs before any HIP call)."""
import ctypes
import os
import random
import shutil
import subprocess
import re

import pytest
import torch

from mlc_decode_amd import _lib
from mlc_decode_amd._lib import MlaDecodeArgs, MlaKvAppendArgs
from mlc_decode_amd.api import get_mla_metadata_host
from oracle import mla_ref as R

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "mla_decode_amd.h")


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\*?\s+\**(mla_[a-z0-9_]+)\(", text, re.M)))


def test_exports_every_declared_symbol(lib):
    declared = header_functions()
    assert len(declared) >= 10
    assert sorted(_lib.EXPORTED) == declared
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.mla_version() == 2
    assert lib.mla_last_error() is not None


def _c_layout(tmp_path, struct, fields):
    """sizeof and offsetof of `fields` as the C compiler lays out `struct` from the header."""
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("%zu\\n", offsetof({struct}, {f}));\n' for f in fields)
    src.write_text(f'#include <stddef.h>\n#include <stdio.h>\n#include "mla_decode_amd.h"\n'
                   f'int main(void) {{\n  printf("%zu\\n", sizeof({struct}));\n{body}  return 0;\n}}\n')
    exe = tmp_path / "layout"
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    subprocess.run(["gcc", "-std=c99", "-I", inc, "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    return [int(v) for v in out]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc to lay out the header's structs")
@pytest.mark.parametrize("cls,name", [(MlaDecodeArgs, "mla_decode_args"),
                                      (_lib.MlaKvAppendArgs, "mla_kv_append_args")])
def test_struct_layout_matches_header(tmp_path, cls, name):
    fields = [f for f, _ in cls._fields_]
    c = _c_layout(tmp_path, name, fields)
    assert c[0] == ctypes.sizeof(cls)
    assert c[1:] == [getattr(cls, f).offset for f in fields]


def test_split_plan_matches_reference_rule(lib):
    ns, bpc, ex = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    for L in (1, 7, 33, 64, 65, 2048, 3000, 4095, 8192, 65536):
        for req in (1, 3, 64, 104, 312):
            for bn in (32, 64):
                for spread in (0, 1):
                    assert lib.mla_split_plan(L, req, bn, spread, ctypes.byref(ns), ctypes.byref(bpc),
                                              ctypes.byref(ex)) == 0
                    assert (ns.value, bpc.value, ex.value) == R.split_plan(L, req, bn, bool(spread))
    assert lib.mla_split_plan(0, 4, 32, 0, ctypes.byref(ns), ctypes.byref(bpc), ctypes.byref(ex)) != 0
    assert b"seqlen_kv" in lib.mla_last_error()


@pytest.mark.parametrize("seed", range(5))
def test_host_schedule_matches_oracle(seed):
    rng = random.Random(100 + seed)
    B = rng.choice([1, 2, 64, 128, 132])
    lengths = [rng.choice([0, 1, 64, 65, rng.randint(1, 16384)]) for _ in range(B)]
    for parts in (1, 5, 128, 256):
        for fo in (0, 5):
            sched, splits = get_mla_metadata_host(lengths, parts, fo)
            recs, prefix = R.schedule_balanced(lengths, parts, fo)
            assert sched[:, :5].tolist() == [list(r) for r in recs]
            assert torch.all(sched[:, 5:] == 0)
            assert splits.tolist() == prefix
        # the default (fixed_overhead < 0): min-payload packing at the default overhead
        sched, splits = get_mla_metadata_host(lengths, parts, -1)
        recs, prefix, _ = R.schedule_min_payload(lengths, parts, _lib.MLA_DEFAULT_SPLIT_OVERHEAD)
        assert sched[:, :5].tolist() == [list(r) for r in recs]
        assert torch.all(sched[:, 5:] == 0)
        assert splits.tolist() == prefix
    for forced in (1, 3, 8):
        sched, splits = get_mla_metadata_host(lengths, 0, forced_splits=forced)
        recs, prefix = R.schedule_forced(lengths, forced)
        assert sched[:, :5].tolist() == [list(r) for r in recs]
        assert splits.tolist() == prefix


def test_workspace_bytes(lib):
    n = lib.mla_workspace_bytes(64, 1, 128, 128)
    slots, rows = 64 + 128, 128
    pad = lambda x: -(-x // 256) * 256  # noqa: E731
    # fp32 lse per (slot, row), one fp32 scale per 128-dim chunk (each padded to 256 bytes),
    # then fp16 partial rows of 512
    assert n == pad(slots * rows * 4) + pad(slots * rows * 16) + slots * rows * 512 * 2
    assert lib.mla_workspace_bytes(0, 1, 16, 4) == 0


@pytest.mark.parametrize("ramp", ["batch_1_to_256", "random", "tiny_steps"])
def test_workspace_growth_keeps_retired_below_live(lib, ramp):
    """A stream's workspace is never freed once handed out, so the buffers it outgrows stay
    alive: their total must stay below the live buffer's size whatever the request sequence
    (a batch ramp at H = 128, random sizes, requests one byte apart)."""
    from mlc_decode_amd.api import grown_workspace_size
    rng = random.Random(7)
    if ramp == "batch_1_to_256":
        needs = [lib.mla_workspace_bytes(b, 1, 128, 256 // 1) + 256 for b in range(1, 257)]
    elif ramp == "random":
        needs = [rng.randrange(256, 1 << 34) for _ in range(2000)]
    else:
        needs = list(range(300, 5000))
    live, retired, grown = None, 0, 0
    for need in needs:
        if live is None or live < need:
            size = grown_workspace_size(live, need)
            assert size >= need and (live is None or size >= 2 * live)
            if live is not None:
                retired += live
            live, grown = size, grown + 1
            assert retired < live
    # the ramp of 256 batch sizes reallocates only a handful of times
    assert grown <= 64 if ramp != "batch_1_to_256" else grown <= 10


@pytest.mark.parametrize("ptrs, ns, needle", [
    ((0, 256, 256, 256, 256, 256, 256), 4, b"NULL"),
    ((256,) * 7, 0, b"ns must be in [1, 128]"),
    ((256,) * 7, 129, b"ns must be in [1, 128]"),
    ((256, 256, 8, 256, 256, 256, 256), 4, b"16-byte aligned"),
])
def test_mla_launch_rejects_bad_args(lib, ptrs, ns, needle):
    # The reference's binding (argtypes [c_void_p] * 7 + [c_int], restype None): an invalid call
    # launches nothing and leaves its reason in mla_last_error.
    assert lib.mla_launch.restype is None
    assert lib.mla_launch(*ptrs, ns) is None
    assert needle in lib.mla_last_error()


def test_num_parts(lib):
    # up to 16 rows: one workgroup per CU whose four waves share one tile; up to 32 rows: four
    # single-wave workgroups per CU; up to 64 rows: one 64-row workgroup per CU; above: one
    # 128-row workgroup per CU, head blocks sharing the CU count
    assert lib.mla_num_parts(1, 1, 16, 1, 256) == 256
    assert lib.mla_num_parts(1, 1, 32, 1, 256) == 1024
    assert lib.mla_num_parts(1, 1, 64, 1, 256) == 256
    assert lib.mla_num_parts(64, 1, 128, 1, 256) == 256
    assert lib.mla_num_parts(32, 2, 128, 1, 256) == 128
    assert lib.mla_num_parts(8, 1, 129, 1, 256) == 128
    assert lib.mla_num_parts(1, 1, 16, 2, 256) < 0


def test_variant_query(lib):
    vals = [ctypes.c_int32() for _ in range(4)]
    ptrs = [ctypes.byref(v) for v in vals]
    assert lib.mla_variant(16, *ptrs) == 0 and [v.value for v in vals] == [4, 1, 1, 16]
    assert lib.mla_variant(32, *ptrs) == 0 and [v.value for v in vals] == [1, 2, 1, 32]
    # above 32 rows the wide kernel runs (MLA_WIDE unset): its latent ring holds 4 stages
    assert lib.mla_variant(64, *ptrs) == 0 and [v.value for v in vals] == [4, 1, 4, 64]
    assert lib.mla_variant(128, *ptrs) == 0 and [v.value for v in vals] == [4, 2, 4, 128]
    assert lib.mla_variant(0, *ptrs) == 1


def _valid_args():
    a = MlaDecodeArgs()
    a.batch, a.s_q, a.heads_q, a.heads_k = 2, 1, 16, 1
    a.dtype, a.causal, a.sm_scale, a.num_blocks = 0, 1, 576 ** -0.5, 4
    base = 1 << 20  # fake, aligned device addresses: validation fails before any use
    a.q_nope, a.q_rope = base, base + 1024
    a.q_stride_b = a.q_rope_stride_b = 16 * 576
    a.q_stride_h = a.q_rope_stride_h = 576
    a.kv_nope, a.kv_rope = base, base + 1024
    a.kv_stride_page = a.kv_rope_stride_page = 64 * 576
    a.kv_stride_tok = a.kv_rope_stride_tok = 576
    a.block_table, a.block_table_stride, a.block_table_width = base, 2, 2
    a.num_parts = 4
    a.cache_seqlens = a.tile_sched = a.num_splits = base
    a.out = base
    a.o_stride_b, a.o_stride_h = 16 * 512, 512
    a.workspace = base
    a.workspace_bytes = 0
    return a


@pytest.mark.parametrize("field,value,code,needle", [
    ("heads_k", 2, 4, b"heads_k"),
    ("dtype", 7, 1, b"dtype"),
    ("batch", 0, 1, b"batch"),
    ("kv_nope", (1 << 20) + 8, 1, b"16-byte"),
    ("kv_stride_tok", 577, 1, b"strides"),
    ("kv_stride_tok", 1 << 24, 4, b"2^24"),
    ("kv_rope_stride_tok", 1 << 25, 4, b"2^24"),
    ("num_parts", 0, 1, b"num_parts"),
    ("sm_scale", 0.0, 1, b"sm_scale"),
    ("workspace_bytes", 0, 2, b"workspace"),
    # the decode is bounded by the block table's width: it must be given, and
    # name columns inside one row
    ("block_table_width", 0, 1, b"block_table_width"),
    ("block_table_width", 3, 1, b"block_table_width"),
    ("block_table_width", -1, 1, b"block_table_width"),
    ("table_reserved", 1, 1, b"table_reserved"),
    ("status", (1 << 20) + 2, 1, b"status"),
])
def test_decode_rejects_bad_args(lib, field, value, code, needle):
    a = _valid_args()
    setattr(a, field, value)
    rc = lib.mla_decode_fwd(ctypes.byref(a), None)
    assert rc == code
    assert needle in lib.mla_last_error()
    with pytest.raises(_lib.MlaError):
        _lib.check("mla_decode_fwd", rc)


@pytest.mark.parametrize("changes,code,needle", [
    (dict(kv_format=2), 1, b"kv_format"),
    (dict(kv_reserved=1), 1, b"kv_format"),
    (dict(kv_format=1, dtype=1), 4, b"bf16"),
    (dict(kv_format=1, block_table=None), 4, b"paged"),
    (dict(kv_format=1), 1, b"kv_scale"),                                   # no scale array
    (dict(kv_format=1, kv_scale=(1 << 20) + 4), 1, b"kv_scale"),            # misaligned
    (dict(kv_format=1, kv_scale=1 << 20, kv_scale_stride_blk=65), 1, b"kv_scale"),
    (dict(kv_format=1, kv_scale=1 << 20, kv_stride_tok=520), 1, b"16 bytes"),
    (dict(kv_format=1, kv_scale=1 << 20, kv_scale_stride_page=256, kv_scale_stride_blk=64,
          kv_stride_tok=512, kv_stride_page=32768), 2, b"workspace"),      # valid up to the workspace
])
def test_decode_rejects_bad_fp8_args(lib, changes, code, needle):
    a = _valid_args()
    for k, v in changes.items():
        setattr(a, k, v)
    rc = lib.mla_decode_fwd(ctypes.byref(a), None)
    assert rc == code
    assert needle in lib.mla_last_error()


def test_decode_noalloc_rejects_workspace_and_oversize(lib):
    # both checks run before any device call
    a = _valid_args()
    assert lib.mla_decode_fwd_noalloc(ctypes.byref(a), None) == 1
    assert b"no workspace" in lib.mla_last_error()
    a.workspace = None
    a.workspace_bytes = 0
    a.batch, a.heads_q, a.num_parts = 512, 128, 1024  # 1.1 GiB of partials
    assert lib.mla_workspace_bytes(512, 1, 128, 1024) > _lib.MLA_NOALLOC_SCRATCH_BYTES
    assert lib.mla_decode_fwd_noalloc(ctypes.byref(a), None) == 2
    assert b"MLA_NOALLOC_SCRATCH_BYTES" in lib.mla_last_error()


@pytest.mark.parametrize("w,v,code,needle", [
    (None, 1 << 20, 1, b"NULL"),
    (1 << 20, None, 1, b"NULL"),
    ((1 << 20) + 8, 1 << 20, 1, b"w_uv_blk"),
    (1 << 20, (1 << 20) + 2, 1, b"4-byte"),
])
def test_combine_absorb_rejects_bad_args(lib, w, v, code, needle):
    a = _valid_args()
    a.workspace_bytes = 1 << 40  # valid decode arguments: the absorb's own checks decide
    rc = lib.mla_combine_absorb(ctypes.byref(a), w, v, None)
    assert rc == code
    assert needle in lib.mla_last_error()
    a.workspace_bytes = 0          # the decode arguments are validated first
    assert lib.mla_combine_absorb(ctypes.byref(a), 1 << 20, 1 << 20, None) == 2


def test_metadata_rejects_bad_args(lib):
    seq = (ctypes.c_int32 * 2)(5, 6)
    sched = (ctypes.c_int32 * 64)()
    splits = (ctypes.c_int32 * 3)()
    assert lib.mla_get_metadata_host(seq, 2, 3, -1, 2, sched, splits) != 0   # parts != B*forced
    assert b"forced_splits" in lib.mla_last_error()
    assert lib.mla_get_metadata_host(seq, 0, 3, -1, 0, sched, splits) != 0
    assert lib.mla_get_metadata(None, 2, 3, -1, 0, None, None, None) != 0


def test_python_api_refuses_cpu_tensors():
    from mlc_decode_amd import MlaKernel, mla_decode_with_kvcache
    k = MlaKernel(1, 16, 1, 64)
    x = torch.zeros(1, 16, 512, dtype=torch.float16)
    with pytest.raises(ValueError):
        k(x, torch.zeros(1, 16, 64, dtype=torch.float16), torch.zeros(1, 64, 1, 512, dtype=torch.float16),
          torch.zeros(1, 64, 1, 64, dtype=torch.float16))
    with pytest.raises(ValueError):
        mla_decode_with_kvcache(torch.zeros(1, 1, 16, 576), torch.zeros(1, 64, 1, 576),
                                torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32))
    with pytest.raises(ValueError):
        MlaKernel(1, 16, 2, 64)


def _valid_append_args():
    a = MlaKvAppendArgs()
    a.batch, a.n_new, a.dtype, a.num_blocks = 2, 1, 0, 8
    base = 1 << 20  # fake, aligned device addresses: validation fails before any use
    a.kv_new = base
    a.new_stride_b, a.new_stride_t = 576, 576
    a.kv_nope, a.kv_rope = base, base + 1024
    a.kv_stride_page = a.kv_rope_stride_page = 64 * 576
    a.kv_stride_tok = a.kv_rope_stride_tok = 576
    a.block_table, a.block_table_stride, a.max_pages = base, 4, 4
    a.cache_seqlens = base
    return a


@pytest.mark.parametrize("field,value,needle", [
    ("batch", 0, b"batch"),
    ("n_new", 0, b"n_new"),
    ("n_new", 65, b"n_new"),
    ("dtype", 3, b"dtype"),
    ("kv_new", None, b"NULL"),
    ("cache_seqlens", None, b"NULL"),
    ("kv_nope", (1 << 20) + 8, b"16-byte"),
    ("new_stride_t", 580, b"strides"),
    ("kv_stride_tok", -8, b"strides"),
    ("max_pages", 0, b"max_pages"),
    ("num_blocks", 0, b"num_blocks"),
])
def test_kv_append_rejects_bad_args(lib, field, value, needle):
    a = _valid_append_args()
    setattr(a, field, value)
    rc = lib.mla_kv_append(ctypes.byref(a), None)
    assert rc == 1
    assert needle in lib.mla_last_error()


def test_kv_append_python_checks():
    from mlc_decode_amd import kv_append
    new = torch.zeros(2, 1, 576, dtype=torch.bfloat16)
    with pytest.raises(ValueError):  # host tensors are refused: there is no CPU path
        kv_append(new, torch.zeros(4, 64, 1, 576, dtype=torch.bfloat16),
                  torch.zeros(2, 2, dtype=torch.int32), torch.zeros(2, dtype=torch.int32))


@pytest.mark.parametrize("changes,code,needle", [
    (dict(indices=1 << 20, topk=64, indices_stride=64, s_q=2), 4, b"s_q"),
    (dict(indices=1 << 20, topk=0, indices_stride=64), 4, b"topk"),
    (dict(indices=1 << 20, topk=4096, indices_stride=4096), 4, b"topk"),
    (dict(indices=1 << 20, topk=64, indices_stride=32), 1, b"indices_stride"),
    # over the fp8 cache (no page table needed): valid up to the workspace check
    (dict(indices=1 << 20, topk=64, indices_stride=64, kv_format=1, kv_scale=1 << 20, block_table=None),
     2, b"workspace"),
    (dict(indices=1 << 20, topk=64, indices_stride=64, block_table=None, cache_seqlens=None), 2, b"workspace"),
])
def test_decode_rejects_bad_sparse_args(lib, changes, code, needle):
    a = _valid_args()
    for k, v in changes.items():
        setattr(a, k, v)
    rc = lib.mla_decode_fwd(ctypes.byref(a), None)
    assert rc == code
    assert needle in lib.mla_last_error()


def test_prepare_w_uv_layout():
    # blk[h, kb, n, kk] = W_UV[h, 32 kb + kk, n]: the k-blocked layout mla_combine_absorb reads
    from mlc_decode_amd.api import prepare_w_uv
    w = torch.arange(3 * 512 * 128, dtype=torch.float32).reshape(3, 512, 128)
    blk = prepare_w_uv(w)
    assert blk.shape == (3, 16, 128, 32) and blk.is_contiguous()
    for h, kb, n, kk in [(0, 0, 0, 0), (1, 3, 77, 5), (2, 15, 127, 31), (2, 7, 0, 31)]:
        assert blk[h, kb, n, kk] == w[h, 32 * kb + kk, n]
    assert torch.equal(blk.transpose(2, 3).reshape(3, 512, 128), w)
    with pytest.raises(ValueError):
        prepare_w_uv(w[:, :, :64])


_PACK32_PROG = r"""
#include <cstdio>
#include <cstdint>
#include "mla_sched.h"
using namespace mla;
int main() {
  uint64_t x = 88172645463325252ull;
  auto rnd = [&](int m) { x ^= x << 13; x ^= x >> 7; x ^= x << 17; return (int)(x % (uint64_t)m); };
  long bad = 0, steps = 0;
  for (int trial = 0; trial < 20000; ++trial) {
    const int f = rnd(8), T = 1 + rnd(trial % 3 == 0 ? 12 : 400);
    PackState st{T, 0, 0};
    int remain = T, part = 0, cum = 0;
    const int B = 1 + rnd(40);
    for (int b = 0; b < B; ++b) {
      const int n = rnd(5) == 0 ? 0 : rnd(trial % 2 ? 30 : 3000);
      const bool ok64 = pack_sequence(b, n, (int64_t)T, f, st, NoEmit{});
      const bool ok32 = pack_sequence32(n, T, f, remain, part, cum);
      ++steps;
      if (ok64 != ok32) { ++bad; break; }
      if (!ok64) break;
      if (st.remain != remain || st.part != part || st.cum != cum) { ++bad; break; }
    }
  }
  std::printf("%ld %ld\n", bad, steps);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++ to build the schedule header")
def test_pack_sequence32_equals_pack_sequence(tmp_path):
    # the device's 32-bit branch-free packing step against the reference step, on random
    # sequences, payloads (including T <= f) and overheads
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = tmp_path / "pack32.cpp"
    src.write_text(_PACK32_PROG)
    exe = tmp_path / "pack32"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(repo, "include"),
                    "-I", os.path.join(repo, "mlc_decode_amd", "csrc"), "-o", str(exe), str(src)], check=True)
    bad, steps = map(int, subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split())
    assert steps > 100000 and bad == 0


_WALK_PROG = r"""
#include <cstdio>
#include <cstdint>
#include <vector>
#include "mla_sched.h"
using namespace mla;
int main() {
  uint64_t x = 0x9E3779B97F4A7C15ull;
  auto rnd = [&](int m) { x ^= x << 13; x ^= x >> 7; x ^= x << 17; return (int)(x % (uint64_t)m); };
  long bad = 0, walked = 0;
  for (int trial = 0; trial < 20000; ++trial) {
    const int B = 1 + (trial % 5 == 0 ? rnd(700) : rnd(140));
    std::vector<int32_t> L(B);
    for (auto& l : L) {
      const int r = rnd(10);
      l = r == 0 ? 0 : r == 1 ? 1 + rnd(64) : trial % 4 == 0 ? rnd(300000) : trial % 4 == 1 ? 4096 : rnd(20000);
    }
    const int parts = 1 + rnd(trial % 3 == 0 ? 8 : 1100), f = rnd(8);
    for (int mp = 0; mp < 2; ++mp) {
      const int nw = (B + kWalkWin - 1) / kWalkWin;
      std::vector<int32_t> pg(B), s1(parts * 8, -7), n1(B + 1, -7), s2(parts * 8, -7), n2(B + 1, -7), S(B + 1);
      std::vector<WalkEntry> ent(8 * nw);
      std::vector<uint64_t> msk(8 * nw);
      schedule_packed(L.data(), B, parts, f, mp, pg.data(), s1.data(), n1.data());
      if (schedule_walk_host(L.data(), B, parts, f, mp, S.data(), ent.data(), msk.data(), s2.data(), n2.data()) < 0)
        continue;
      ++walked;
      if (s1 != s2 || n1 != n2) ++bad;
    }
  }
  std::printf("%ld %ld\n", bad, walked);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++ to build the schedule header")
def test_walk_schedule_equals_serial_packing(tmp_path):
    # the closed form between resets (the device's parallel schedule, emulated on the host with
    # the same windows, entries and masks) against the serial greedy packing, on random
    # batches with empty and one-page sequences, tiny payloads (c = T - f < 1) and f = 0 .. 7
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = tmp_path / "walk.cpp"
    src.write_text(_WALK_PROG)
    exe = tmp_path / "walk"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(repo, "include"),
                    "-I", os.path.join(repo, "mlc_decode_amd", "csrc"), "-o", str(exe), str(src)], check=True)
    bad, walked = map(int, subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split())
    assert walked > 30000 and bad == 0
