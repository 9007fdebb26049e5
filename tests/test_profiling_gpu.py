"""GPU tests of ferrite.profiling (reference: tests/test_profiling.py:20-34): event timing of a
HIP kernel, the kernel report of flash attention (its HIP kernels are listed as this
library's), and a trace with device activity."""

import json

import pytest
import torch

from ferrite.kernels import flash_attention, matmul
from ferrite.profiling import compile_report, timeit, trace

pytestmark = pytest.mark.gpu


def test_timeit_and_kernel_report(dev, tmp_path):
    x = torch.ones(256, 256, device=dev, dtype=torch.bfloat16)
    t = timeit(lambda a: matmul(a, a), x, warmup=1, iters=3, events=True)
    assert t.median_s > 0 and t.iters == 3
    q = torch.randn(1, 2, 256, 64, device=dev, dtype=torch.bfloat16)
    rep = compile_report(lambda a: flash_attention(a, a, a, causal=True), q, name="attn", dump_dir=str(tmp_path))
    assert rep["n_ferrite_kernels"] >= 1 and any("attn_fwd" in k for k in rep["ferrite_kernels"]), rep
    assert (tmp_path / "attn.kernels.txt").read_text().count("ferrite") >= 1


def test_trace_writes_a_profile(dev, tmp_path):
    with trace(str(tmp_path / "t")):
        x = torch.ones(64, 64, device=dev, dtype=torch.bfloat16)
        matmul(x, x)
    data = json.loads((tmp_path / "t" / "trace.json").read_text())
    names = [e.get("name", "") for e in data["traceEvents"]]
    assert any("gemm" in n for n in names), names[:20]
