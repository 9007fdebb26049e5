"""The bench.py contract that needs no GPU: more than one GPU is refused with a message and exit
code 2 (this build measures one GPU), and the committed traffic table that feeds the roofline's
`traffic` field parses into plausible byte counts."""

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="4")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_traffic_table_feeds_the_roofline():
    sys.path.insert(0, ROOT)
    import bench

    for kernel in ("attn_fwd", "add_rmsnorm"):
        t = bench._traffic(kernel)
        assert t is not None and t > 0
    # the forward's algorithmic bytes: q, k, v read and O written (4 B H S D 2) plus lse (4 B H S)
    alg = 4 * 4 * 16 * 2048 * 128 * 2 + 4 * 16 * 2048 * 4
    assert 1.0 <= bench._traffic("attn_fwd") / alg < 2.0
    flops = 4 * 4 * 16 * 2048 * 2048 * 128 * 0.5
    roof = bench._roofline("attn_fwd", flops, alg, flops / 900e12, traffic=bench._traffic("attn_fwd"))
    assert roof["bound"] == "mfma" and abs(roof["frac"] - 900.0 / 2516.6) < 1e-3
    assert roof["unit"] == "TFLOP/s" and abs(roof["achieved"] - 900.0) < 0.01 and roof["traffic"] > alg
    # a traffic figure read from the committed profile says where it came from
    assert "profiles/hbm_traffic.md" in roof["traffic_source"] and "not measured in this run" in roof["traffic_source"]
    norm = bench._roofline("add_rmsnorm", 5 * 4096 * 1024, 33556480, 33556480 / 5000e9)
    assert norm["bound"] == "hbm" and norm["unit"] == "GB/s" and abs(norm["frac"] - 5000 / 8000) < 1e-4
    # without a traffic figure the field is left out rather than reported as null
    assert "traffic" not in norm and "traffic_source" not in norm
    json.dumps(roof)


def test_cpu_baseline_legs_shape():
    """cpu_baseline carries the headline (attention forward) and a leg per other BASELINE kernel,
    each in its kernel's unit with the threads used; run here with a tiny time budget."""
    sys.path.insert(0, ROOT)
    import bench

    cb = bench.cpu_baseline(budget_s=0.05)
    assert cb["unit"] == "TFLOP/s" and cb["kind"] == "port" and cb["value"] > 0 and cb["cores"] >= 1
    legs = cb["legs"]
    assert set(legs) == {"add_rmsnorm", "matmul_bf16_4096", "matmul_f32_1000"}
    assert legs["add_rmsnorm"]["unit"] == "GB/s" and legs["add_rmsnorm"]["cores"] == 1
    for leg in legs.values():
        assert leg["value"] > 0 and leg["sample"]
    json.dumps(cb)
