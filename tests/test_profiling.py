"""Tests of ferrite.profiling (reference: tests/test_profiling.py:9-34): roofline math off
the device (CPU), and timing, the kernel report and a trace (CPU here, GPU in
test_profiling_gpu.py)."""

import json

import pytest
import torch

from ferrite import platform
from ferrite.kernels.matmul import matmul_flops
from ferrite.profiling import analyze, compile_report, format_table, timeit, trace


def test_roofline_math_off_device():
    peaks = platform.peaks("MI355X")
    assert peaks.cores == 256 and peaks.ridge_point > 100
    p = analyze("mm", flops=2 * 4096**3, bytes_=3 * 4096 * 4096 * 2, seconds=110e-6, peaks=peaks)
    assert p.bound == "compute" and 0 < p.percent_of_roof < 100
    assert abs(p.percent_of_roof - 100 * (2 * 4096**3 / 2.5166e15) / 110e-6) < 1e-9
    q = analyze("norm", flops=5 * 4096 * 1024, bytes_=4 * 4096 * 1024 * 2, seconds=6.75e-6, peaks=peaks)
    assert q.bound == "memory" and abs(q.percent_of_roof - 100 * q.bytes / 8.0e12 / 6.75e-6) < 1e-9
    f32 = analyze("mm32", flops=2e9, bytes_=12e6, seconds=50e-6, peaks=peaks, peak_flops=peaks.fp32_flops)
    assert f32.ridge == peaks.fp32_flops / peaks.hbm_bytes_per_s
    table = format_table([p, q])
    assert "| kernel |" in table and "| mm |" in table and "memory" in table
    assert set(p.to_dict()) >= {"achieved_tflops", "achieved_gbps", "bound", "percent_of_roof"}
    assert analyze("x", 1, 1, 1, peaks=None).bound in ("unknown", "compute", "memory")


def test_timeit_report_and_trace_on_cpu(tmp_path):
    x = torch.ones(256, 256)
    t = timeit(lambda a: a @ a, x, warmup=1, iters=3)
    assert t.median_s > 0 and t.iters == 3 and t.min_s <= t.median_s
    rep = compile_report(lambda a: a @ a, x, name="mm", dump_dir=str(tmp_path))
    assert rep["n_kernels"] == 0 and (tmp_path / "mm.kernels.txt").exists()  # no GPU: no device kernels
    with trace(str(tmp_path / "t")):
        (x @ x).sum()
    data = json.loads((tmp_path / "t" / "trace.json").read_text())
    assert data["traceEvents"]
    assert matmul_flops(256, 256, 256) == 2 * 256**3
