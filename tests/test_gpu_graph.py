"""A serving step captured in a HIP graph (torch.cuda.CUDAGraph): append the step's new tokens
to the paged cache, schedule, decode.  Every replay is compared bit for bit with the same step
run eagerly from a copy of the same state, with eager work and synchronisations between the
replays (the library records no memset nodes and allocates nothing once its workspace exists)."""
import sys

import pytest
import torch

from mlc_decode_amd import (flash_mla_with_kvcache, get_mla_metadata, kv_append, mla_decode_absorbed,
                            prepare_w_uv, quantize_kv_cache)

pytestmark = pytest.mark.gpu

B, H, PAGES = 4, 64, 8   # 8 pages (512 tokens) reserved per sequence


def say(msg):
    print(f"[gpu-graph] {msg}", flush=True)
    sys.stdout.flush()


def state(seed, fp8=False):
    g = torch.Generator().manual_seed(seed)
    nb = B * PAGES
    kv = (torch.randn(nb, 64, 1, 576, generator=g)).to(torch.bfloat16).cuda()
    if fp8:
        kv = quantize_kv_cache(kv)
    table = torch.randperm(nb, generator=g).reshape(B, PAGES).to(torch.int32).cuda()
    lens = torch.tensor([0, 63, 200, 447], dtype=torch.int32).cuda()
    return kv, table, lens


def clone_cache(kv):
    if isinstance(kv, torch.Tensor):
        return kv.clone()
    return type(kv)(*(t.clone() for t in kv))


def cache_equal(a, b):
    if isinstance(a, torch.Tensor):
        return torch.equal(a, b)
    return all(torch.equal(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize("fp8", [False, True])
def test_captured_append_schedule_decode(gpu, fp8):
    kv, table, lens = state(1, fp8)
    q = torch.empty(B, 1, H, 576, dtype=torch.bfloat16, device="cuda")
    new = torch.empty(B, 1, 576, dtype=torch.bfloat16, device="cuda")
    g = torch.Generator().manual_seed(2)

    def step(kv_, lens_):
        kv_append(new, kv_, table, lens_)
        sched, splits = get_mla_metadata(lens_, H, 1)
        return flash_mla_with_kvcache(q, kv_, table, lens_, 512, sched, splits, causal=True)

    # eager warm-up on a throw-away copy: creates the workspace, loads the library
    q.copy_(torch.randn(B, 1, H, 576, generator=g).to(torch.bfloat16))
    new.copy_(torch.randn(B, 1, 576, generator=g).to(torch.bfloat16))
    step(clone_cache(kv), lens.clone())
    torch.cuda.synchronize()

    say(f"capture fp8={fp8}")
    graph = torch.cuda.CUDAGraph()
    kv_before = clone_cache(kv)
    lens_before = lens.clone()
    with torch.cuda.graph(graph):
        out_g, lse_g = step(kv, lens)
    # capture records the work without running it: the state is unchanged
    torch.cuda.synchronize()
    assert cache_equal(kv, kv_before) and torch.equal(lens, lens_before)

    for rep in range(3):
        q.copy_(torch.randn(B, 1, H, 576, generator=g).to(torch.bfloat16))
        new.copy_(torch.randn(B, 1, 576, generator=g).to(torch.bfloat16))
        kv_e, lens_e = clone_cache(kv), lens.clone()
        torch.cuda.synchronize()
        say(f"replay {rep} fp8={fp8}")
        graph.replay()
        torch.cuda.synchronize()
        out_e, lse_e = step(kv_e, lens_e)   # the same step, eagerly, from the same state
        torch.cuda.synchronize()
        assert torch.equal(lens, lens_e) and lens.cpu().tolist() == (lens_before.cpu() + rep + 1).tolist()
        assert cache_equal(kv, kv_e), f"replay {rep}: cache differs"
        assert torch.equal(out_g, out_e), f"replay {rep}: out differs"
        assert torch.equal(lse_g, lse_e), f"replay {rep}: lse differs"


def test_captured_absorbed_decode(gpu):
    kv, table, lens = state(3)
    q = torch.empty(B, 1, H, 576, dtype=torch.bfloat16, device="cuda")
    g = torch.Generator().manual_seed(4)
    w_blk = prepare_w_uv((torch.randn(H, 512, 128, generator=g) * 512 ** -0.5).to(torch.bfloat16).cuda())
    lens.copy_(torch.tensor([1, 64, 300, 511], dtype=torch.int32))

    def step():
        sched, splits = get_mla_metadata(lens, H, 1)
        return mla_decode_absorbed(q, kv, table, lens, sched, splits, w_blk, causal=True)

    q.copy_(torch.randn(B, 1, H, 576, generator=g).to(torch.bfloat16))
    step()
    torch.cuda.synchronize()
    say("capture absorbed")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        v_g, lse_g = step()
    for rep in range(3):
        q.copy_(torch.randn(B, 1, H, 576, generator=g).to(torch.bfloat16))
        torch.cuda.synchronize()
        say(f"replay absorbed {rep}")
        graph.replay()
        torch.cuda.synchronize()
        v_e, lse_e = step()
        torch.cuda.synchronize()
        assert torch.equal(v_g, v_e) and torch.equal(lse_g, lse_e), f"replay {rep} differs"


def test_graph_replay_after_workspace_growth(gpu):
    """A graph captured on a stream keeps writing into the workspace it was captured with after a
    later eager call on that stream needed a larger one: the old buffer is retired, never
    freed, so a tensor allocated afterwards (the guard) cannot alias it."""
    from mlc_decode_amd import mla_decode_with_kvcache
    kv, table, lens = state(5)
    g = torch.Generator().manual_seed(6)
    q = torch.randn(B, 1, H, 576, generator=g).to(torch.bfloat16).cuda()
    s = torch.cuda.Stream()

    def step():
        sched, splits = get_mla_metadata(lens, H, 1)
        return flash_mla_with_kvcache(q, kv, table, lens, 512, sched, splits, causal=True)

    with torch.cuda.stream(s):
        out_ref, lse_ref = step()          # creates the workspace of stream s
    torch.cuda.synchronize()
    say("capture on a user stream")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out_g, lse_g = step()
    torch.cuda.synchronize()
    # a much larger decode on the same stream grows its workspace (B=64, H=128: ~84 MB)
    Bb, Hb, Lb = 64, 128, 256
    qb = torch.randn(Bb, 1, Hb, 576, generator=g).to(torch.bfloat16).cuda()
    kvb = torch.randn(Bb * 4, 64, 1, 576, generator=g).to(torch.bfloat16).cuda()
    tb = torch.arange(Bb * 4, dtype=torch.int32).reshape(Bb, 4).cuda()
    lb = torch.full((Bb,), Lb, dtype=torch.int32).cuda()
    say("grow the workspace eagerly on the same stream")
    with torch.cuda.stream(s):
        mla_decode_with_kvcache(qb, kvb, tb, lb)
    torch.cuda.synchronize()
    guard = torch.full((96 << 20,), 7, dtype=torch.uint8, device=gpu)
    for rep in range(3):
        say(f"replay after growth {rep}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_ref) and torch.equal(lse_g, lse_ref), f"replay {rep} differs"
        assert bool(torch.all(guard == 7)), f"replay {rep} wrote outside its workspace"
