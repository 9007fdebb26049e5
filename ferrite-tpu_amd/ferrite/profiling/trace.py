"""Capture a host + device trace viewable in Perfetto or chrome://tracing.

Reference: src/ferrite/profiling/trace.py (``jax.profiler`` xplane traces). Here
torch's profiler records host operations and, on a ROCm GPU, every HIP kernel
with its measured duration, this library's kernels among them; the trace is
written as ``<logdir>/trace.json``.
"""

from __future__ import annotations

import contextlib
import os

import torch


@contextlib.contextmanager
def trace(logdir: str, create_perfetto_link: bool = False):
    """``with trace("traces/run1"): ...`` records host and device activity into logdir/trace.json.
    ``create_perfetto_link`` is accepted for the reference's signature; open the file at
    https://ui.perfetto.dev instead."""
    os.makedirs(logdir, exist_ok=True)
    acts = [torch.profiler.ProfilerActivity.CPU]
    if torch.cuda.is_available():
        acts.append(torch.profiler.ProfilerActivity.CUDA)
    prof = torch.profiler.profile(activities=acts, acc_events=True)
    prof.__enter__()
    try:
        yield logdir
    finally:
        if torch.cuda.is_available() and torch.cuda.is_initialized():
            torch.cuda.synchronize()
        prof.__exit__(None, None, None)
        prof.export_chrome_trace(os.path.join(logdir, "trace.json"))
