"""What a call launched on the GPU: this library's kernels, library GEMMs, torch kernels, copies.

Reference: src/ferrite/profiling/hlo.py (``compile_report``: fusions, Pallas custom calls,
collectives and XLA's cost model in the optimised HLO). There is no XLA here: the
counterpart of "what did the compiler make of this function" is the list of kernels
the call actually launches, taken from one profiled run, with their device times.
"""

from __future__ import annotations

import os
import re

import torch


def _kind(name: str) -> str:
    if name.startswith("_ZN7ferrite") or "ferrite::" in name:
        return "ferrite"
    if name.startswith("Cijk_") or "gemm" in name.lower() or "hipblaslt" in name.lower():
        return "library_gemm"
    if "copy" in name.lower() or "Memcpy" in name or "Memset" in name or "fillBuffer" in name:
        return "copy"
    return "torch"


def compile_report(fn, *args, name: str = "fn", dump_dir: str | None = None, **kw) -> dict:
    """Run ``fn(*args, **kw)`` once to warm up and once under the profiler; summarise the
    device kernels it launched (``n_ferrite_kernels`` is the counterpart of the reference's
    ``n_pallas_calls``). With ``dump_dir``, writes ``<name>.kernels.txt``, one kernel a line."""
    fn(*args, **kw)
    if torch.cuda.is_available() and torch.cuda.is_initialized():
        torch.cuda.synchronize()
    acts = [torch.profiler.ProfilerActivity.CPU]
    if torch.cuda.is_available():
        acts.append(torch.profiler.ProfilerActivity.CUDA)
    with torch.profiler.profile(activities=acts, acc_events=True) as prof:
        fn(*args, **kw)
        if torch.cuda.is_available() and torch.cuda.is_initialized():
            torch.cuda.synchronize()
    kernels = []
    for ev in prof.events():
        if str(getattr(ev, "device_type", "")).endswith("CUDA") and getattr(ev, "device_time", 0) is not None:
            kernels.append((ev.name, float(getattr(ev, "device_time", 0.0))))
    counts = {"ferrite": 0, "library_gemm": 0, "copy": 0, "torch": 0}
    times = dict.fromkeys(counts, 0.0)
    for kname, us in kernels:
        k = _kind(kname)
        counts[k] += 1
        times[k] += us
    report = {
        "name": name,
        "n_kernels": len(kernels),
        "n_ferrite_kernels": counts["ferrite"],
        "n_library_gemms": counts["library_gemm"],
        "n_copies": counts["copy"],
        "n_torch_kernels": counts["torch"],
        "device_time_us": {k: round(v, 3) for k, v in times.items()},
        "ferrite_kernels": sorted({re.sub(r"\(.*", "", k) for k, _ in kernels if _kind(k) == "ferrite"}),
    }
    if dump_dir:
        os.makedirs(dump_dir, exist_ok=True)
        with open(os.path.join(dump_dir, f"{name}.kernels.txt"), "w") as f:
            for kname, us in kernels:
                f.write(f"{us:10.3f} us  {_kind(kname):12s}  {kname}\n")
        report["dump_dir"] = dump_dir
    return report
