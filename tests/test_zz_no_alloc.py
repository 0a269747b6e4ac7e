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


_CAPTURE_SCRIPT = r'''
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
from mlc_decode_amd import _lib
from mlc_decode_amd.api import get_mla_metadata_host, make_decode_args
from mlc_decode_amd.inputs import MlaConfig, make_inputs

lib = _lib.load()
cfg = MlaConfig("noalloc_graph", batch=6, s_q=1, heads=128, dtype=torch.bfloat16, sigma=1.0,
                seqlen_groups=[(1, L) for L in [3000, 64, 1, 4100, 700, 2049]])
inp = make_inputs(cfg, seed=5)
# the schedule on the host, so that no kernel of the library runs before the capture: the
# first call of the library in this process (code-object load, scratch lookup) is captured
sched, splits = get_mla_metadata_host(inp.cache_seqlens.tolist(), 256)
d = inp.to("cuda:0")
sched, splits = sched.cuda(), splits.cuda()
out = torch.full((6, 1, 128, 512), float("nan"), dtype=torch.bfloat16, device="cuda:0")
lse = torch.full((6, 128, 1), float("nan"), dtype=torch.float32, device="cuda:0")
args, _, _, keep = make_decode_args(d.q, d.kv_cache, d.block_table, d.cache_seqlens, sched, splits,
                                    inp.sm_scale, True, out=out, lse=lse)
args.workspace, args.workspace_bytes = None, 0
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
with torch.cuda.graph(graph, stream=side):
    rc = lib.mla_decode_fwd_noalloc(ctypes.byref(args), ctypes.c_void_p(side.cuda_stream))
assert rc == 0, lib.mla_last_error()
print("captured the first call", flush=True)
# the reference: the workspace entry point, eagerly, after the capture
ref_args, ref_out, ref_lse, keep2 = make_decode_args(d.q, d.kv_cache, d.block_table, d.cache_seqlens,
                                                     sched, splits, inp.sm_scale, True)
assert lib.mla_decode_fwd(ctypes.byref(ref_args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
torch.cuda.synchronize()
assert int(splits[-1].item()) > 6, "the case must have split sequences (partials in the scratch)"
junk = torch.randn(1 << 20, device="cuda:0")
for r in range(3):
    out.fill_(float("nan"))
    lse.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out), f"replay {r}: outputs differ"
    assert torch.equal(lse, ref_lse), f"replay {r}: lse differs"
    junk.mul_(1.0001).add_(0.5)   # eager work between the replays
    torch.cuda.synchronize()
    print(f"replay {r} bit-identical", flush=True)
'''


def test_noalloc_first_call_under_graph_capture(gpu, tmp_path):
    """The allocation-free entry point's first call in a process made inside a HIP graph capture
    (the library's code object and the scratch address are looked up during capture), then
    three replays, each compared bit for bit with mla_decode_fwd run eagerly.  Runs in a fresh
    process so that nothing has called the library before the capture."""
    import os
    import subprocess
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "capture_first.py"
    script.write_text(_CAPTURE_SCRIPT)
    _say("noalloc: first call inside graph capture (fresh process)")
    proc = subprocess.run([sys.executable, "-u", str(script), repo], capture_output=True, text=True,
                          timeout=240, cwd=repo)
    print(proc.stdout[-2000:], proc.stderr[-2000:])
    assert proc.returncode == 0, proc.stderr[-2000:]
    assert proc.stdout.count("bit-identical") == 3
