"""MLA decode benchmark on one MI355X (headline metric: µs per call at B=64, H=128, L=4096, bf16).

A step is one decode call over the whole batch with inputs resident in HBM and the tile
schedule computed beforehand (it is computed once per decode step and shared by every
layer).  Prints ONE JSON line with the metric, the roofline of the dominant kernel (the
split-KV main kernel, timed with HIP events on the launch stream), the same fraction for the
whole call, the end-to-end time with the schedule included, the fraction of a measured
stream peak, cold-cache times, and the CPU oracle timed on the host cores as a baseline.

    python bench.py [--steps K] [--warmup W] [--config C2] [--no-cpu-baseline]
    python bench.py --stream-probe          # achievable HBM bandwidth of plain stream ops
    python bench.py --all-configs [--record mla_best_configs_mi355x.json]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_PEAK_TFLOPS = 2500.0   # dense bf16 / fp16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline")
    ap.add_argument("--all-configs", action="store_true", help="also print one line per config to stderr")
    ap.add_argument("--record", default="", metavar="PATH",
                    help="with --all-configs: write the per-config record (tile, splits, timings, "
                         "roofline) as JSON, the MI355X counterpart of mla_best_configs.json")
    ap.add_argument("--append", action="store_true",
                    help="measure the paged KV-cache append (mla_kv_append) at every config's "
                         "batch and s_q instead of the decode; one JSON line per config")
    ap.add_argument("--sparse", action="store_true",
                    help="measure the sparse (top-k = 2048) decode on synthetic index lists; one JSON "
                         "line per shape")
    ap.add_argument("--absorb", action="store_true",
                    help="time the fused combine + absorbed W_UV projection against combine + bmm")
    ap.add_argument("--kv-fp8", action="store_true",
                    help="measure the decode over the fp8 (e4m3) latent cache at every config (bf16 "
                         "queries); one JSON line per config")
    ap.add_argument("--stream-probe", action="store_true",
                    help="print the achievable HBM bandwidth of plain stream ops (fill, copy, add, "
                         "sum over 1 GiB tensors) and exit")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache timings")
    ap.add_argument("--no-probe", action="store_true",
                    help="skip the stream probe (profiling runs: keeps its copies out of the trace)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run a plain MIB-MiB device copy 3x (scale for FETCH/WRITE_SIZE counters)")
    ap.add_argument("--windows", type=int, default=5,
                    help="timing windows of --steps calls each; every figure is their median")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_gpu(fn, steps, warmup, stream):
    from mlc_decode_amd.timing import time_gpu as _time_gpu
    return _time_gpu(fn, steps, warmup, stream)


WINDOWS = 5  # timing windows per figure; the median is reported (set by --windows)


def time_windows(fn, steps, warmup, stream, windows=None):
    """ms per call in each of ``windows`` windows of exactly ``steps`` calls (HIP events on
    ``stream``, a synchronisation on both sides of every window); ``warmup`` untimed calls
    before the first."""
    n = WINDOWS if windows is None else windows
    return [time_gpu(fn, steps, warmup if i == 0 else 0, stream) for i in range(n)]


def median(xs):
    import statistics
    return statistics.median(xs)


def settle_clocks(fn, stream, seconds=0.25):
    from mlc_decode_amd.timing import settle_clocks as _settle
    _settle(fn, stream, seconds)


FLUSH_BYTES = 1 << 30  # larger than the L2s and the 256 MB MALL together


def time_cold(fn, reps, stream, dirty=False):
    """Median ms of single calls, each after a 1 GiB sweep that evicts the caches.  The default
    sweep reads (a sum), so the caches hold clean lines; with ``dirty`` it writes (a fill), so
    the call's first misses also pay for writing back the dirty lines the fill left in L2 and
    MALL.  The sweep runs long enough for the host to queue the call behind it, so the GPU does
    not wait on the host between the two events."""
    import statistics

    import torch
    junk = torch.ones(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda:0")
    fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        if dirty:
            junk.fill_(1)
        else:
            junk.sum()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        fn()
        e.record(stream)
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    del junk
    return statistics.median(times)


def stream_probe(reps=20):
    """Achievable HBM bandwidth of plain stream ops over 1 GiB tensors (GB/s of algorithmic
    traffic, 10^9 bytes): the denominator of a measured-peak fraction, as the reference's
    scripts/bandwidth_probe.py:52-71 measures its own device."""
    import torch
    n = FLUSH_BYTES // 2
    x = torch.randn(n, dtype=torch.bfloat16, device="cuda:0")
    y = torch.empty_like(x)
    a = torch.randn(n, dtype=torch.bfloat16, device="cuda:0")
    out = torch.empty_like(x)
    nb = n * 2
    cases = {
        "fill_w": (lambda: y.fill_(1.0), nb),
        "copy_rw": (lambda: y.copy_(x), 2 * nb),
        "add_2r1w": (lambda: torch.add(x, a, out=out), 3 * nb),
        "sum_r": (lambda: x.sum(dtype=torch.float32), nb),
    }
    res = {}
    stream = torch.cuda.current_stream()
    for name, (fn, traffic) in cases.items():
        ms = time_gpu(fn, reps, 3, stream)
        res[name] = round(traffic / (ms * 1e-3) / 1e9, 1)
    del x, y, a, out
    torch.cuda.empty_cache()
    res["best"] = max(res.values())
    return res


PEAK_SCLK_MHZ = 2400.0  # MI355X peak engine clock, at which the 2.5 PFLOP/s dense bf16 figure holds


def mfma_probe(iters=100000):
    """Dense bf16 MFMA rate the device sustains (eight independent 16x16x32 chains per wave,
    two waves per SIMD on every CU) and the shader clock measured during it (clock64 against
    the wall clock): the MFMA counterpart of the stream probe, and the clock that scales the
    spec peak (2.5 PFLOP/s at 2400 MHz) to this run."""
    import ctypes
    import statistics

    import torch
    from mlc_decode_amd.build import PROBE_PATH
    lib = ctypes.CDLL(PROBE_PATH)
    lib.mla_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.mla_probe_mfma.restype = ctypes.c_int
    lib.mla_probe_wall_clock_khz.restype = ctypes.c_int
    props = torch.cuda.get_device_properties(0)
    wgs = 2 * props.multi_processor_count
    sink = torch.empty(wgs * 256 * 4, dtype=torch.float32, device="cuda:0")
    clocks = torch.zeros(wgs * 4, dtype=torch.int64, device="cuda:0")
    stream = torch.cuda.current_stream()
    run = lambda n: lib.mla_probe_mfma(n, sink.data_ptr(), clocks.data_ptr(), wgs, stream.cuda_stream)  # noqa: E731
    if run(iters // 10) != 0:
        raise RuntimeError("mfma probe launch failed")
    torch.cuda.synchronize()
    times = []
    for _ in range(3):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        run(iters)
        e.record(stream)
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    ms = statistics.median(times)
    flops = wgs * 4 * iters * 8 * 2 * 16 * 16 * 32
    c = clocks.view(wgs, 4).cpu().double()
    wall_khz = lib.mla_probe_wall_clock_khz()
    ratio = ((c[:, 2] - c[:, 0]) / (c[:, 3] - c[:, 1]).clamp(min=1)).median().item()
    sclk = ratio * wall_khz / 1e3 if wall_khz > 0 else None
    tflops = flops / (ms * 1e-3) / 1e12
    return {"tflops": round(tflops, 1), "sclk_mhz": None if sclk is None else round(sclk, 1),
            "wall_clock_khz": wall_khz,
            "peak_at_clock_tflops": None if sclk is None else round(MFMA_PEAK_TFLOPS * sclk / PEAK_SCLK_MHZ, 1),
            "probe": f"{wgs} workgroups x 4 waves x {iters} rounds of 8 independent v_mfma_f32_16x16x32_bf16, "
                     "median of 3 launches"}


FP8_TOKEN_BYTES = 512 + 64 * 2 + 4 * 4  # e4m3 latent codes, bf16 rope, four fp32 block scales


def measure(cfg_name, steps, warmup, kv_fp8=False, cold=True):
    import dataclasses

    import torch
    from mlc_decode_amd import _lib
    from mlc_decode_amd.api import flash_mla_with_kvcache, get_mla_metadata, quantize_kv_cache
    from mlc_decode_amd.inputs import CONFIGS, algorithmic_bytes, algorithmic_flops, make_inputs

    cfg = CONFIGS[cfg_name]
    if kv_fp8 and cfg.dtype != torch.bfloat16:
        cfg = dataclasses.replace(cfg, dtype=torch.bfloat16)  # the fp8 cache takes bf16 queries
    cpu_inp = make_inputs(cfg, seed=0)
    inp = cpu_inp.to("cuda:0")
    kv = quantize_kv_cache(inp.kv_cache) if kv_fp8 else inp.kv_cache
    B, s_q, H = cfg.batch, cfg.s_q, cfg.heads
    stream = torch.cuda.current_stream()
    forced = cfg.num_splits or 0
    sched, splits = get_mla_metadata(inp.cache_seqlens, s_q * H, 1, forced_splits=forced)
    out = torch.empty(B, s_q, H, 512, dtype=cfg.dtype, device="cuda:0")
    lse = torch.empty(B, H, s_q, dtype=torch.float32, device="cuda:0")

    import ctypes
    from mlc_decode_amd._lib import check
    from mlc_decode_amd.api import make_decode_args
    lib = _lib.load()
    args, _, _, keep = make_decode_args(inp.q, kv, inp.block_table, inp.cache_seqlens,
                                        sched, splits, inp.sm_scale, inp.causal, out, lse)
    ap = ctypes.byref(args)
    sp = stream.cuda_stream

    def call():  # the public call path, validation and all
        flash_mla_with_kvcache(inp.q, kv, inp.block_table, inp.cache_seqlens, 512,
                               sched, splits, softmax_scale=inp.sm_scale, causal=inp.causal,
                               out=out, lse=lse)

    settle_clocks(call, stream)
    win_call = time_windows(call, steps, warmup, stream)
    ms_call = median(win_call)
    # the two kernels separately, launched through the C ABI on the same stream
    win_main = time_windows(lambda: check("mla_splitkv_fwd", lib.mla_splitkv_fwd(ap, sp)),
                            steps, warmup, stream)
    ms_main = median(win_main)
    ms_combine = median(time_windows(lambda: check("mla_combine_fwd", lib.mla_combine_fwd(ap, sp)),
                                     steps, warmup, stream))
    ms_meta = median(time_windows(lambda: get_mla_metadata(inp.cache_seqlens, s_q * H, 1, forced_splits=forced),
                                  steps, warmup, stream))

    def end_to_end():  # the schedule computed in the call, then the decode on it
        sc, sp_ = get_mla_metadata(inp.cache_seqlens, s_q * H, 1, forced_splits=forced)
        flash_mla_with_kvcache(inp.q, kv, inp.block_table, inp.cache_seqlens, 512,
                               sc, sp_, softmax_scale=inp.sm_scale, causal=inp.causal,
                               out=out, lse=lse)

    ms_e2e = median(time_windows(end_to_end, steps, warmup, stream))
    ms_cold = None if not cold else time_cold(call, max(10, min(steps, 40)), stream)
    ms_cold_dirty = None if not cold else time_cold(call, max(10, min(steps, 40)), stream, dirty=True)
    del keep

    nbytes = algorithmic_bytes(cpu_inp.cache_seqlens, B, s_q, H, 2)
    if kv_fp8:  # KV at FP8_TOKEN_BYTES per cached token instead of 576 bf16 values
        nbytes -= int(cpu_inp.cache_seqlens.sum()) * (576 * 2 - FP8_TOKEN_BYTES)
    flops = algorithmic_flops(cpu_inp.cache_seqlens, s_q, H, cfg.causal)
    t_hbm = nbytes / (HBM_PEAK_GBS * 1e9)
    t_mfma = flops / (MFMA_PEAK_TFLOPS * 1e12)
    bound = "hbm" if t_hbm >= t_mfma else "mfma"
    gbs = nbytes / (ms_main * 1e-3) / 1e9
    tflops = flops / (ms_main * 1e-3) / 1e12
    n_splits = int(splits[-1].item())
    # the same roofline over the whole call (main kernel, combine and the gap between them)
    call_frac = (nbytes / (ms_call * 1e-3) / 1e9 / HBM_PEAK_GBS if bound == "hbm"
                 else flops / (ms_call * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS)
    return dict(cfg=cfg, cpu_inp=cpu_inp, ms_call=ms_call, ms_main=ms_main, ms_combine=ms_combine,
                windows_call=win_call, windows_main=win_main,
                ms_meta=ms_meta, ms_e2e=ms_e2e, ms_cold=ms_cold, ms_cold_dirty=ms_cold_dirty,
                nbytes=nbytes, flops=flops,
                bound=bound, gbs=gbs, tflops=tflops, call_frac=call_frac,
                parts=int(sched.shape[0]), n_splits=n_splits)


SPARSE_SHAPES = {  # name: (batch, heads, topk, tokens per sequence)
    "S1": (64, 128, 2048, 8192),   # DeepSeek-V3.2-style top-2048 over 8K contexts, all heads
    "S2": (128, 16, 2048, 8192),   # the same per TP-8 rank
}


def measure_sparse(name, steps, warmup, kv_fp8=False):
    """Sparse decode: each sequence owns tokens_per_seq / 64 random pages of the pool and its
    top-k list is a random choice of distinct tokens among them."""
    import torch
    from mlc_decode_amd.api import flash_mla_with_kvcache, get_mla_metadata, quantize_kv_cache
    B, H, topk, per_seq = SPARSE_SHAPES[name]
    g = torch.Generator().manual_seed(0)
    pages = per_seq // 64
    nb = B * pages
    kv = torch.randn(nb, 64, 1, 576, generator=g).to(torch.bfloat16).cuda()
    if kv_fp8:
        kv = quantize_kv_cache(kv)
    q = torch.randn(B, 1, H, 576, generator=g).to(torch.bfloat16).cuda()
    table = torch.randperm(nb, generator=g).reshape(B, pages)
    idx = torch.empty(B, 1, topk, dtype=torch.int32)
    for b in range(B):
        t = torch.randperm(per_seq, generator=g)[:topk]
        idx[b, 0] = (table[b, t // 64] * 64 + t % 64).to(torch.int32)
    idx = idx.cuda()
    lens = torch.zeros(B, dtype=torch.int32, device="cuda")
    sched, splits = get_mla_metadata(lens, H, 1, topk=topk)
    out = torch.empty(B, 1, H, 512, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B, H, 1, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    def call():
        flash_mla_with_kvcache(q, kv, None, None, 512, sched, splits, softmax_scale=576 ** -0.5,
                               out=out, lse=lse, indices=idx)

    settle_clocks(call, stream)
    ms = time_gpu(call, steps, warmup, stream)
    token_bytes = FP8_TOKEN_BYTES if kv_fp8 else 576 * 2
    nbytes = B * topk * (token_bytes + 4) + B * H * (576 + 512) * 2 + B * H * 4
    flops = 2 * B * H * topk * (576 + 512)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"op": "decode_sparse_fp8_cache" if kv_fp8 else "decode_sparse", "shape": name, "batch": B, "heads": H, "topk": topk,
            "us_call": round(ms * 1e3, 2), "algorithmic_bytes": nbytes, "tbps": round(gbs / 1e3, 3),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "parts": int(sched.shape[0]), "splits": int(splits[-1].item()),
            "note": "call = main + combine through the Python API; indices random distinct tokens "
                    "of each sequence's pages"}


def measure_absorb(cfg_name, steps, warmup):
    """Absorbed value projection v = o . W_UV per head after the decode: the fused kernel
    (combine merged into the product's prologue, ``mla_combine_absorb``) against the unfused
    pair (combine kernel, then torch's batched product).  Weights are random N(0, 1/512)."""
    import ctypes

    import torch
    from mlc_decode_amd import _lib
    from mlc_decode_amd._lib import check
    from mlc_decode_amd.api import get_mla_metadata, make_decode_args, prepare_w_uv
    from mlc_decode_amd.inputs import CONFIGS, make_inputs

    cfg = CONFIGS[cfg_name]
    inp = make_inputs(cfg, seed=0).to("cuda:0")
    B, s_q, H = cfg.batch, cfg.s_q, cfg.heads
    M = B * s_q
    g = torch.Generator().manual_seed(1)
    w_uv = (torch.randn(H, 512, 128, generator=g) * 512 ** -0.5).to(cfg.dtype).cuda()
    w_t = prepare_w_uv(w_uv)
    sched, splits = get_mla_metadata(inp.cache_seqlens, s_q * H, 1, forced_splits=cfg.num_splits or 0)
    out = torch.empty(B, s_q, H, 512, dtype=cfg.dtype, device="cuda:0")
    lse = torch.empty(B, H, s_q, dtype=torch.float32, device="cuda:0")
    v = torch.empty(B, s_q, H, 128, dtype=cfg.dtype, device="cuda:0")
    lib = _lib.load()
    args, _, _, keep = make_decode_args(inp.q, inp.kv_cache, inp.block_table, inp.cache_seqlens,
                                        sched, splits, inp.sm_scale, inp.causal, out, lse)
    ap = ctypes.byref(args)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    check("mla_splitkv_fwd", lib.mla_splitkv_fwd(ap, sp))  # partials and single-split rows in place

    def fused():
        check("mla_combine_absorb", lib.mla_combine_absorb(ap, w_t.data_ptr(), v.data_ptr(), sp))

    def unfused():
        check("mla_combine_fwd", lib.mla_combine_fwd(ap, sp))
        torch.matmul(out.view(M, H, 512).transpose(0, 1), w_uv)

    settle_clocks(fused, stream)
    ms_fused = time_gpu(fused, steps, warmup, stream)
    ms_unfused = time_gpu(unfused, steps, warmup, stream)
    torch.cuda.synchronize()
    del keep
    n = (splits[1:] - splits[:-1]).cpu()
    rows = s_q * H
    part_bytes = int(sum(rows * (1024 if k == 1 else k * (1024 + 4)) for k in n.tolist()))
    nbytes = H * 128 * 512 * 2 + part_bytes + M * H * 128 * 2
    flops = 2 * M * H * 512 * 128
    gbs = nbytes / (ms_fused * 1e-3) / 1e9
    return {"op": "combine_absorb", "config": cfg_name, "rows": M, "heads": H,
            "us_fused": round(ms_fused * 1e3, 2), "us_combine_then_bmm": round(ms_unfused * 1e3, 2),
            "algorithmic_bytes": nbytes, "tbps": round(gbs / 1e3, 3), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tflops": round(flops / (ms_fused * 1e-3) / 1e12, 1), "splits": int(splits[-1].item()),
            "note": "bytes = W_UV + split partials (or the single-split row) + v; decode not timed"}


def cpu_baseline(m, budget_s):
    """The fp32 CPU oracle (the reference's torch decode, restated in oracle/) on a bounded
    sample of the same workload's sequences, scaled to microseconds per full call."""
    import torch
    from oracle import mla_ref as R
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    inp = m["cpu_inp"]
    B = inp.q.shape[0]
    idx = [0]
    R.decode_paged(inp.q[:1], inp.kv_cache, inp.block_table[:1], inp.cache_seqlens[:1],
                   inp.sm_scale, inp.causal)  # warm-up
    t0 = time.perf_counter()
    R.decode_paged(inp.q[:1], inp.kv_cache, inp.block_table[:1], inp.cache_seqlens[:1],
                   inp.sm_scale, inp.causal)
    per_seq = max(time.perf_counter() - t0, 1e-6)
    n = max(1, min(B, int(budget_s / 3 / per_seq)))
    idx = list(range(n))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        R.decode_paged(inp.q[idx], inp.kv_cache, inp.block_table[idx], inp.cache_seqlens[idx],
                       inp.sm_scale, inp.causal)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[1]
    tok_sample = int(inp.cache_seqlens[idx].sum())
    tok_all = int(inp.cache_seqlens.sum())
    us_full = med * 1e6 * tok_all / max(tok_sample, 1)
    return {"value": round(us_full, 1), "unit": "us/call", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{n} of {B} sequences ({tok_sample} of {tok_all} cached tokens), median of 3, "
                      f"scaled by token count; fp32 torch on {cpu_model()}"}


def measure_append(cfg_name, steps):
    """mla_kv_append of s_q new tokens per sequence into the config's paged cache (two spare
    pages per sequence, so `steps` successive appends stay inside the table)."""
    import torch
    from mlc_decode_amd.api import kv_append
    from mlc_decode_amd.inputs import CONFIGS, make_inputs
    cfg = CONFIGS[cfg_name]
    inp = make_inputs(cfg, seed=0)
    B, n_new = cfg.batch, cfg.s_q
    nb = inp.kv_cache.shape[0]
    spare = torch.arange(nb, nb + 2 * B, dtype=torch.int32).view(B, 2)
    lens = inp.cache_seqlens.clone()
    P = int(((lens + 63) // 64).max()) + 2
    bt = torch.zeros(B, P, dtype=torch.int32)
    for b in range(B):
        n = (int(lens[b]) + 63) // 64
        bt[b, :n] = inp.block_table[b, :n]
        bt[b, n:n + 2] = spare[b]
    cache = torch.zeros(nb + 2 * B, 64, 1, 576, dtype=cfg.dtype, device="cuda:0")
    cache[:nb] = inp.kv_cache.to("cuda:0")
    new = torch.randn(B, n_new, 576).to(cfg.dtype).to("cuda:0")
    btg, lg = bt.to("cuda:0"), lens.to("cuda:0")
    steps = min(steps, 64 // n_new)
    stream = torch.cuda.current_stream()
    import ctypes
    from mlc_decode_amd import _lib
    args = kv_append(new, cache, btg, lg)
    torch.cuda.synchronize()
    steps = (steps - 1) // 2
    ms = time_gpu(lambda: kv_append(new, cache, btg, lg), steps, 0, stream)
    lib, ap, sp = _lib.load(), ctypes.byref(args), stream.cuda_stream
    ms_c = time_gpu(lambda: _lib.check("mla_kv_append", lib.mla_kv_append(ap, sp)), steps, 0, stream)
    nbytes = B * n_new * 576 * 2 * 2 + B * 4 * 2  # rows read + written, lengths read + written
    return {"op": "kv_append", "config": cfg_name, "batch": B, "n_new": n_new,
            "us_call": round(ms * 1e3, 3), "us_c_abi": round(ms_c * 1e3, 3), "bytes": nbytes,
            "gbs": round(nbytes / (ms_c * 1e-3) / 1e9, 2),
            "note": "launch-bound: a few hundred KB per call; us_call is the Python API, us_c_abi "
                    "the C entry point with its arguments prepared once"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if args.stream_probe:
        print(json.dumps({"op": "stream_probe", "unit": "GB/s", "bytes_per_tensor": FLUSH_BYTES,
                          **stream_probe()}), flush=True)
        return
    if args.append:
        for name in ("C1", "C2", "C3", "C4", "C5"):
            print(json.dumps(measure_append(name, args.steps)), flush=True)
        return
    if args.sparse:
        for name in SPARSE_SHAPES:
            print(json.dumps(measure_sparse(name, args.steps, args.warmup, kv_fp8=args.kv_fp8)), flush=True)
        return
    if args.absorb:
        for name in ("C1", "C2", "C3", "C4", "C5"):
            print(json.dumps(measure_absorb(name, args.steps, args.warmup)), flush=True)
        return
    if args.kv_fp8:
        for name in ("C1", "C2", "C3", "C4", "C5"):
            mm = measure(name, args.steps, args.warmup, kv_fp8=True, cold=False)
            frac = (mm["gbs"] / HBM_PEAK_GBS) if mm["bound"] == "hbm" else (mm["tflops"] / MFMA_PEAK_TFLOPS)
            print(json.dumps({"op": "decode_fp8_cache", "config": name, "us_call": round(mm["ms_call"] * 1e3, 2),
                              "us_main": round(mm["ms_main"] * 1e3, 2),
                              "us_combine": round(mm["ms_combine"] * 1e3, 2),
                              "algorithmic_bytes": mm["nbytes"], "tbps": round(mm["gbs"] / 1e3, 3),
                              "tflops": round(mm["tflops"], 1), "bound": mm["bound"],
                              "roofline_frac": round(frac, 4), "parts": mm["parts"],
                              "splits": mm["n_splits"]}), flush=True)
        return
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    global WINDOWS
    WINDOWS = max(1, args.windows)
    probe = None if args.no_probe else stream_probe()
    mprobe = None if args.no_probe else mfma_probe()
    m = measure(args.config, args.steps, args.warmup, cold=not args.no_cold)
    cfg = m["cfg"]
    if args.all_configs:
        from mlc_decode_amd import _lib
        from mlc_decode_amd.api import kernel_variant
        record = {"device": torch.cuda.get_device_name(0), "arch": "gfx950",
                  "command": "python bench.py " + " ".join(sys.argv[1:]),
                  "peaks": {"hbm_gbs": HBM_PEAK_GBS, "mfma_bf16_tflops": MFMA_PEAK_TFLOPS,
                            "stream_probe_gbs": probe, "mfma_probe": mprobe},
                  "configs": {}}
        for name in ("C1", "C2", "C3", "C4", "C5"):
            mm = m if name == args.config else measure(name, max(20, args.steps // 4), 5, cold=not args.no_cold)
            c = mm["cfg"]
            frac = (mm["gbs"] / HBM_PEAK_GBS) if mm["bound"] == "hbm" else (mm["tflops"] / MFMA_PEAK_TFLOPS)
            entry = {"us_call": round(mm["ms_call"] * 1e3, 2), "us_main": round(mm["ms_main"] * 1e3, 2),
                     "us_combine": round(mm["ms_combine"] * 1e3, 2),
                     "us_metadata": round(mm["ms_meta"] * 1e3, 2),
                     "us_end_to_end": round(mm["ms_e2e"] * 1e3, 2),
                     "us_call_cold": None if mm["ms_cold"] is None else round(mm["ms_cold"] * 1e3, 2),
                     "us_call_cold_dirty": None if mm["ms_cold_dirty"] is None else round(mm["ms_cold_dirty"] * 1e3, 2),
                     "call_frac": round(mm["call_frac"], 4),
                     "tbps": round(mm["gbs"] / 1e3, 3), "tflops": round(mm["tflops"], 1),
                     "bound": mm["bound"], "roofline_frac": round(frac, 4),
                     "mfma_frac_of_clock_peak": (round(mm["tflops"] / mprobe["peak_at_clock_tflops"], 4)
                                                 if mprobe and mprobe["peak_at_clock_tflops"] else None),
                     "hbm_frac_of_measured_peak": round(mm["gbs"] / probe["best"], 4) if probe else None,
                     "parts": mm["parts"], "splits": mm["n_splits"]}
            print(json.dumps({"config": name, **entry}), file=sys.stderr, flush=True)
            record["configs"][name] = {
                "shape": {"batch": c.batch, "s_q": c.s_q, "heads": c.heads, "seqlen": c.seqlen,
                          "dtype": "bf16" if c.dtype == torch.bfloat16 else "fp16",
                          "causal": c.causal},
                "splits_policy": (f"forced {c.num_splits}" if c.num_splits
                                  else f"min-payload, overhead {_lib.MLA_DEFAULT_SPLIT_OVERHEAD} pages"),
                "tile": kernel_variant(c.s_q * c.heads), **entry}
        if args.record:
            with open(args.record, "w") as f:
                json.dump(record, f, indent=1)
                f.write("\n")
    peak = HBM_PEAK_GBS if m["bound"] == "hbm" else MFMA_PEAK_TFLOPS
    achieved = m["gbs"] if m["bound"] == "hbm" else m["tflops"]
    traffic = None
    tfile = os.path.join(REPO, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    line = {
        "metric": "MLA decode us/call (B=64,H=128,L=4096)",
        "value": round(m["ms_call"] * 1e3, 3),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["ms_call"], 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp16",
        "data": "synthetic (seeded N(0,1) q and paged latent cache, random block table)",
        "config": {"workload": f"{cfg.name}: MLA decode B={cfg.batch} s_q={cfg.s_q} H={cfg.heads} "
                               f"d_qk=576 d_v=512 page=64", "batch": cfg.batch, "s_q": cfg.s_q,
                   "heads": cfg.heads, "seq_len": cfg.seqlen, "parts": m["parts"],
                   "splits": m["n_splits"]},
        "hbm_tbps": round(m["gbs"] / 1e3, 3),
        "mfma_tflops": round(m["tflops"], 2),
        "main_kernel_us": round(m["ms_main"] * 1e3, 3),
        "combine_us": round(m["ms_combine"] * 1e3, 3),
        "metadata_us": round(m["ms_meta"] * 1e3, 3),
        "us_end_to_end_with_metadata": round(m["ms_e2e"] * 1e3, 3),
        "us_call_cold": None if m["ms_cold"] is None else round(m["ms_cold"] * 1e3, 3),
        "us_call_cold_dirty": None if m["ms_cold_dirty"] is None else round(m["ms_cold_dirty"] * 1e3, 3),
        "call_roofline_frac": round(m["call_frac"], 4),
        "stream_probe_gbs": probe,
        "timing": f"median of {WINDOWS} windows of {args.steps} calls each",
        "windows_us_call": [round(x * 1e3, 3) for x in m["windows_call"]],
        "windows_us_main": [round(x * 1e3, 3) for x in m["windows_main"]],
        "mfma_probe": mprobe,
        # MFMA utilisation of the main kernel against the spec peak scaled to the measured clock
        # (reported for every config; the binding fraction for the MFMA-bound ones)
        "mfma_frac_of_clock_peak": (round(m["tflops"] / mprobe["peak_at_clock_tflops"], 4)
                                    if mprobe and mprobe["peak_at_clock_tflops"] else None),
        "mfma_frac_of_measured_peak": round(m["tflops"] / mprobe["tflops"], 4) if mprobe else None,
        "frac_of_measured_peak": (round(m["gbs"] / probe["best"], 4) if m["bound"] == "hbm" and probe else
                                  round(m["tflops"] / mprobe["tflops"], 4) if m["bound"] == "mfma" and mprobe
                                  else None),
        "call_frac_of_measured_peak": (round(m["nbytes"] / (m["ms_call"] * 1e-3) / 1e9 / probe["best"], 4)
                                       if m["bound"] == "hbm" and probe else None),
        "roofline": {"bound": m["bound"], "achieved": round(achieved, 2), "peak": peak,
                     "unit": "GB/s" if m["bound"] == "hbm" else "TFLOP/s",
                     "frac": round(achieved / peak, 4), "traffic": traffic,
                     "algorithmic_bytes": m["nbytes"], "algorithmic_flops": m["flops"]},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(m, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
