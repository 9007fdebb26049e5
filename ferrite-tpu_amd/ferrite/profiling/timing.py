"""Timing with device synchronisation.

Reference: src/ferrite/profiling/timing.py (wall clock around each call, after
``block_until_ready``). Here the wait is ``torch.cuda.synchronize()``; with
``events=True`` each call is bracketed by HIP events on the current stream
instead, which leaves the host's launch latency out.
"""

from __future__ import annotations

import dataclasses
import time

import numpy as np
import torch


@dataclasses.dataclass(frozen=True)
class Timing:
    median_s: float
    min_s: float
    mean_s: float
    std_s: float
    iters: int

    @property
    def median_ms(self) -> float:
        return self.median_s * 1e3


def _sync():
    if torch.cuda.is_available() and torch.cuda.is_initialized():
        torch.cuda.synchronize()


def timeit(fn, *args, warmup: int = 2, iters: int = 10, events: bool = False, **kw) -> Timing:
    """Time ``fn(*args, **kw)``; the first ``warmup`` calls are discarded."""
    for _ in range(warmup):
        fn(*args, **kw)
    _sync()
    samples = []
    for _ in range(iters):
        if events:
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            fn(*args, **kw)
            end.record()
            end.synchronize()
            samples.append(start.elapsed_time(end) * 1e-3)
        else:
            t = time.perf_counter()
            fn(*args, **kw)
            _sync()
            samples.append(time.perf_counter() - t)
    s = np.asarray(samples)
    return Timing(float(np.median(s)), float(s.min()), float(s.mean()), float(s.std()), iters)
