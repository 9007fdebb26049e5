"""Host-side logic of the library checked on the CPU with g++: the C ABI's device resolution
(csrc/device_select.h) and the attention kernels' schedules (csrc/attn_sched.h).

Device resolution.

An entry point works on its stream's device, not on the calling thread's current
device: the CU count that shapes a grid, a kernel's LDS limit and the address of
the allocation-free entry's scratch array are all looked up for the device the
stream belongs to, and per-device one-time set-up runs once under std::call_once
(an XLA FFI handler may be called from several threads with any device current).
The host-side logic is
compiled with g++ against stand-in lookups and run here; on the GPU the same code
runs with hipStreamGetDevice / hipGetDevice behind it.
"""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_device_select_host_logic(tmp_path):
    exe = tmp_path / "device_select_test"
    src = os.path.join(HERE, "cpp", "device_select_test.cpp")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-pthread", src, "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    assert "all checks passed" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_attention_schedules(tmp_path):
    """The CPU replay of every attention launcher's schedule (tests/cpp/attn_schedule_test.cpp):
    grid orders, the split kernels' shares, ring loads, waits and reads from the kernels' own
    schedule header, over lengths 64..4096 (and 8192) and several head counts: every output row
    written once, every ring read served by a completed load of the right tile, no region refilled
    under a reader; and every planted schedule mistake caught."""
    exe = tmp_path / "attn_schedule_test"
    src = os.path.join(HERE, "cpp", "attn_schedule_test.cpp")
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", src, "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-4000:]
    assert "all checks passed" in out.stdout
