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
    """Bounds and fractions from closed forms at MI355X peaks."""
    from ferrite.profiling.roofline import MI355X_MFMA_PEAKS, traffic_bytes

    peaks = platform.peaks("MI355X")
    assert peaks.cores == 256 and peaks.ridge_point > 100
    # bf16 4096^3 in 110 us: matrix floor 54.6 us, HBM floor 12.6 us -> MFMA-bound at 49.6%
    p = analyze("mm", flops=2 * 4096**3, bytes_=3 * 4096 * 4096 * 2, seconds=110e-6, peaks=peaks)
    assert p.bound == "mfma"
    assert abs(p.frac - (2 * 4096**3 / 2.5166e15) / 110e-6) < 1e-12
    assert abs(p.bench_fields()["achieved"] - round(2 * 4096**3 / 110e-6 / 1e12, 2)) < 1e-9
    # add+RMSNorm 4096x1024 in 6.75 us: HBM-bound, frac = bytes / 8 TB/s / time
    q = analyze("norm", flops=5 * 4096 * 1024, bytes_=4 * 4096 * 1024 * 2, seconds=6.75e-6, peaks=peaks,
                traffic=1.004 * 4 * 4096 * 1024 * 2)
    assert q.bound == "hbm" and abs(q.frac - q.bytes / 8.0e12 / 6.75e-6) < 1e-12
    f = q.bench_fields()
    assert f["unit"] == "GB/s" and f["peak"] == 8000.0 and abs(q.excess_traffic - 1.004) < 1e-12
    # fp32 work is priced against the fp32 matrix peak: 2 GFLOP over 12 MB is MFMA-bound there
    f32 = analyze("mm32", flops=2e9, bytes_=12e6, seconds=50e-6, peaks=peaks, precision="fp32")
    assert f32.mfma_peak == MI355X_MFMA_PEAKS["fp32"] and f32.bound == "mfma"
    assert abs(f32.frac - 2e9 / 157.3e12 / 50e-6) < 1e-12
    # the same work at the bf16 peak would be HBM-bound: the precision decides
    assert analyze("mm32", 2e9, 12e6, 50e-6, peaks=peaks).bound == "hbm"
    # the counter calibration: a 256 MiB copy reads back as 256 MiB each way
    assert traffic_bytes(131072, 262144) == 2 * 256 * 2**20
    table = format_table([p, q])
    assert "| kernel |" in table and "| mm |" in table and "| hbm |" in table and "1.004" in table
    assert set(p.to_dict()) >= {"tflops", "gbs", "bound", "frac", "excess_traffic"}
    none = analyze("x", 1, 1, 1, peaks=None)
    assert none.bound in ("unknown", "mfma", "hbm")


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
