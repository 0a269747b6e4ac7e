"""GPU timing used by ``bench.py`` and the check CLI: HIP events recorded on the stream the
work is queued on, around back-to-back calls, after an untimed clock-settling run."""
from __future__ import annotations

import time
from typing import Callable, Optional

import torch


def settle_clocks(fn: Callable[[], object], stream: Optional[torch.cuda.Stream] = None,
                  seconds: float = 0.25) -> None:
    """Run ``fn`` back to back for about ``seconds`` before anything is timed.

    A freshly idle GPU needs tens of milliseconds of load before its clocks settle: the first
    200-call window measured cold reads ~10% slower than the next ones, whatever is timed.
    """
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 1
    while time.perf_counter() - t0 < seconds:
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        n = min(n * 2, 256)


def time_gpu(fn: Callable[[], object], steps: int, warmup: int,
             stream: Optional[torch.cuda.Stream] = None) -> float:
    """Milliseconds per call of ``fn``: ``warmup`` untimed calls, then ``steps`` calls between
    two events recorded on ``stream`` (torch's current stream by default)."""
    if stream is None:
        stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / max(steps, 1)
