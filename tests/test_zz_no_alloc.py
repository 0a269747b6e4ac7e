"""The allocation-free decode (mla_decode_fwd_noalloc) against mla_decode_fwd, through the C ABI.

Two calls in a row on one GPU, the second smaller than the first: the static scratch keeps
the first call's partials, and the second must not depend on them.  The same kernels run in
both entry points, so outputs and LSEs must match bit for bit.
"""
import ctypes
import sys

import pytest
import torch

from mlc_decode_amd import _lib
from mlc_decode_amd.api import get_mla_metadata, make_decode_args
from mlc_decode_amd.inputs import MlaConfig, make_inputs

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _decode_both(cfg, seed, device):
    lib = _lib.load()
    inp = make_inputs(cfg, seed=seed).to(device)
    sched, splits = get_mla_metadata(inp.cache_seqlens, cfg.s_q * cfg.heads, 1)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # the existing entry point, with a workspace the Python layer allocates
    args, out_ref, lse_ref, keep = make_decode_args(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                                    sched, splits, inp.sm_scale, inp.causal)
    assert lib.mla_decode_fwd(ctypes.byref(args), stream) == 0, lib.mla_last_error()
    # the allocation-free one: the same arguments without a workspace
    out = torch.full_like(out_ref, float("nan"))
    lse = torch.full_like(lse_ref, float("nan"))
    args2, _, _, keep2 = make_decode_args(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                          sched, splits, inp.sm_scale, inp.causal, out=out, lse=lse)
    args2.workspace = None
    args2.workspace_bytes = 0
    assert lib.mla_decode_fwd_noalloc(ctypes.byref(args2), stream) == 0, lib.mla_last_error()
    torch.cuda.synchronize()
    return out_ref, lse_ref, out, lse, int(splits[-1].item()), (keep, keep2)


def test_noalloc_matches_decode_fwd(gpu):
    cases = [
        # large first: multi-split sequences over 128 heads fill most of a 64 MiB scratch region
        MlaConfig("noalloc_big", batch=24, s_q=1, heads=128, dtype=torch.bfloat16, sigma=1.0,
                  seqlen_groups=[(1, L) for L in [5000, 4096, 1, 64, 65, 3000, 2048, 777] * 3]),
        # then smaller, fewer heads, fp16, s_q = 2
        MlaConfig("noalloc_small", batch=3, s_q=2, heads=16, dtype=torch.float16, sigma=1.0,
                  seqlen_groups=[(1, 300), (1, 9000), (1, 2)]),
    ]
    for i, cfg in enumerate(cases):
        _say(f"noalloc {cfg.name} B={cfg.batch} s_q={cfg.s_q} H={cfg.heads}")
        out_ref, lse_ref, out, lse, slots, _ = _decode_both(cfg, 70 + i, gpu)
        assert slots > cfg.batch, "the case must have split sequences (partials in the scratch)"
        assert torch.equal(out, out_ref), f"{cfg.name}: outputs differ"
        assert torch.equal(torch.isnan(lse), torch.isnan(lse_ref)) and torch.equal(
            lse.nan_to_num(), lse_ref.nan_to_num()), f"{cfg.name}: lse differs"
