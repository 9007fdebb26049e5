#!/usr/bin/env python
"""Benchmark of ferrite's MI355X kernels on BASELINE.json's metric.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Prints ONE JSON line. `value` is the headline: causal flash-attention forward
throughput (algorithmic TFLOP/s, causal-skipped work counted free as in the
reference's attention_flops) at B=4, H=16, T=2048, d=128 bf16. A "step" is
one forward pass over that batch; K steps are timed back to back with HIP
events on the stream the kernels run on, with inputs resident in HBM. The same
line carries every other kernel of the path under "kernels": attention
backward (delta, dK/dV, dQ), the long-context variant (B=1, H=8, T=8192, d=64),
head dim 256 (B=4, H=8, T=2048, d=256), fused add+RMSNorm ([4096,1024] bf16,
timed over 24 rotating buffer sets so the
working set exceeds the 256 MB Infinity Cache) and the blocked matmul (bf16
4096^3, f32 1000^3). Each carries its roofline fraction against MI355X peaks.
"gpt_train_step" times the caller of these kernels: one forward+backward+AdamW
step of the 12-layer GPT of BASELINE config 5 (bf16 parameters, batch 8 x 1024).
"decode_attention" and "serving" time the serving side: the decode-attention
kernel over a full 8192-key cache, and greedy generation at the reference's
serving-benchmark config (TTFT, inter-token latency).

cpu_baseline: the CPU oracle (numpy f32, the reference's materialised
impl='xla' math) timed on this host's cores on a bounded sample of the same
forward workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ferrite-tpu_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "flash-attn fwd/bwd TFLOP/s + add-RMSNorm GB/s, % of MI355X roofline"
PEAK_BF16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.md")


def _events_time(fn, iters: int, warmup: int) -> float:
    """Average seconds per call of `fn` over `iters` back-to-back calls (HIP events on the current stream)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e-3 / iters


def _settle(fn, seconds: float = 0.2) -> None:
    """Run `fn` back to back for `seconds` before anything is timed. The shader clock needs a
    few milliseconds of sustained load to reach its steady value; without this the first
    kernel measured would be timed partly at the idle clock."""
    import time

    import torch

    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(32):
            fn()
        torch.cuda.synchronize()


# Where `roofline.traffic` comes from: the counters cannot run inside the timed bench (rocprofv3
# --pmc is a run of its own), so the line carries the calibrated figure of the committed summary
# and says so in `traffic_source`.
TRAFFIC_SOURCE = ("profiles/hbm_traffic.md: rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE runs of "
                  "bench.py (one counter per run, calibrated against a 256 MiB copy); read from that "
                  "file, not measured in this run")


def _traffic(kernel: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE), read from the committed summary."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 4 and cells[0] == kernel:
            try:
                return float(cells[3])
            except ValueError:
                return None
    return None


def _roofline(name: str, flops: float, nbytes: float, seconds: float, precision: str = "bf16", traffic=None) -> dict:
    """The bench line's roofline object for one launch (ferrite.profiling.roofline at MI355X peaks)."""
    from ferrite import platform
    from ferrite.profiling.roofline import analyze

    fields = analyze(name, flops, nbytes, seconds, peaks=platform.MI355X, precision=precision,
                     traffic=traffic).bench_fields()
    if traffic is None:
        del fields["traffic"]
    else:
        fields["traffic_source"] = TRAFFIC_SOURCE
    return fields


def bench_attention(b, h, t, d, steps, warmup, seed=7):
    import torch

    from ferrite import _hip
    from ferrite.kernels import attention_flops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    q, k, v, do = (torch.randn(b, h, t, d, device=dev, generator=g).to(torch.bfloat16) for _ in range(4))
    o = torch.empty_like(q)
    lse = torch.empty(b, h, t, device=dev)
    delta = torch.empty(b, h, t, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    scale = d**-0.5
    lib, st, bf = _hip.lib(), _hip.stream_of(q), _hip.BF16
    P = [x.data_ptr() for x in (q, k, v, o, lse, delta, do, dq, dk, dv)]
    qp, kp, vp, op, lp, dp, dop, dqp, dkp, dvp = P
    # The split kernels' exchange buffers (zero bytes where the long-context split does not
    # apply), zero-filled once, as flash_attention() keeps them: one for the forward, one that
    # the backward's dQ and dK/dV take turns with.
    ws_bytes = int(lib.ferrite_hip_attn_fwd_workspace(b, h, t, t, d, bf, 1))
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    wsp = ws.data_ptr() if ws_bytes > 0 else None
    bws_bytes = int(lib.ferrite_hip_attn_bwd_workspace(b, h, t, t, d, bf, 1))
    bws = torch.zeros(max(bws_bytes, 1), dtype=torch.uint8, device=dev)
    bwa = (bws.data_ptr(), bws_bytes) if bws_bytes > 0 else (None, 0)

    def fwd():
        _hip.check(lib.ferrite_hip_attn_fwd_ex(qp, kp, vp, op, lp, b, h, t, t, d, bf, 1, scale, wsp, ws_bytes, st),
                   "fwd")

    def dlt():
        _hip.check(lib.ferrite_hip_attn_bwd_delta(op, dop, dp, b, h, t, d, bf, st), "delta")

    def dkv():
        _hip.check(lib.ferrite_hip_attn_bwd_dkv_ex(qp, kp, vp, dop, lp, dp, dkp, dvp, b, h, t, t, d, bf, 1, scale,
                                                   *bwa, st), "dkv")

    def dqk():
        _hip.check(lib.ferrite_hip_attn_bwd_dq_ex(qp, kp, vp, dop, lp, dp, dqp, b, h, t, t, d, bf, 1, scale, *bwa, st),
                   "dq")

    def dq_delta():
        _hip.check(lib.ferrite_hip_attn_bwd_dq_delta_ex(qp, kp, vp, op, dop, lp, dp, dqp, b, h, t, t, d, bf, 1, scale,
                                                        *bwa, st), "dq_delta")

    def bwd():  # the backward flash_attention runs: dQ computing delta, then dK/dV reading it
        dq_delta()
        dkv()

    def bwd_split():  # the reference's order: delta pass, dK/dV, dQ
        dlt()
        dkv()
        dqk()

    _settle(fwd)
    t_fwd = _events_time(fwd, steps, warmup)
    t_delta = _events_time(dlt, steps, warmup)
    t_dkv = _events_time(dkv, steps, warmup)
    t_dq = _events_time(dqk, steps, warmup)
    t_dq_delta = _events_time(dq_delta, steps, warmup)
    t_bwd_split = _events_time(bwd_split, steps, warmup)
    t_bwd = _events_time(bwd, steps, warmup)
    f_fwd = attention_flops(b, h, t, t, d, causal=True)
    f_bwd = attention_flops(b, h, t, t, d, causal=True, backward=True)
    return {
        "shape": [b, h, t, d], "fwd_key_split": ws_bytes > 0, "bwd_key_split": bws_bytes > 0,
        "fwd_us": t_fwd * 1e6, "fwd_tflops": f_fwd / t_fwd / 1e12,
        "delta_us": t_delta * 1e6, "dkv_us": t_dkv * 1e6, "dq_us": t_dq * 1e6, "dq_with_delta_us": t_dq_delta * 1e6,
        "bwd_split_us": t_bwd_split * 1e6,
        "bwd_us": t_bwd * 1e6, "bwd_tflops": f_bwd / t_bwd / 1e12,
        "fwd_bwd_tflops": (f_fwd + f_bwd) / (t_fwd + t_bwd) / 1e12,
        "fwd_frac_bf16_peak": f_fwd / t_fwd / 1e12 / PEAK_BF16_TFLOPS,
        "bwd_frac_bf16_peak": f_bwd / t_bwd / 1e12 / PEAK_BF16_TFLOPS,
        "flops_fwd": f_fwd, "flops_bwd": f_bwd, "bytes_fwd": 4 * b * h * t * d * 2 + 4 * b * h * t,
    }


def bench_attention_fwd_parts(steps, warmup, seed=11):
    """The headline forward (causal 4x16x2048x128: 512 workgroups of 256 query rows, two rounds on
    256 CUs) beside two workloads that take away one of its costs each, so the gap to peak splits
    into parts measured by this file:
      noncausal:  the same shape without the mask (the non-causal kernel, 128-row tiles, two
                  workgroups per CU): every query tile sweeps all 32 key tiles, so there are no
                  diagonal stages and all tiles are equally long (no tail of short sweeps);
      one_round:  causal 2x16x2048x128: 256 workgroups, one per CU, all resident at once: no second
                  round of workgroups, and the longest tile (32 key tiles) sets the time."""
    import torch

    from ferrite import _hip
    from ferrite.kernels import attention_flops

    dev = torch.device("cuda:0")
    lib, bf = _hip.lib(), _hip.BF16
    rows = {}
    for name, (b, h, t, d, causal) in {"causal": (4, 16, 2048, 128, 1), "noncausal": (4, 16, 2048, 128, 0),
                                       "one_round": (2, 16, 2048, 128, 1)}.items():
        g = torch.Generator(device=dev).manual_seed(seed)
        q, k, v = (torch.randn(b, h, t, d, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
        o, lse = torch.empty_like(q), torch.empty(b, h, t, device=dev)
        st = _hip.stream_of(q)

        def fwd(q=q, k=k, v=v, o=o, lse=lse, b=b, h=h, t=t, d=d, causal=causal, st=st):
            _hip.check(lib.ferrite_hip_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                                lse.data_ptr(), b, h, t, t, d, bf, causal, d**-0.5, st), "fwd")

        _settle(fwd, 0.1)
        sec = _events_time(fwd, steps, warmup)
        fl = attention_flops(b, h, t, t, d, causal=bool(causal))
        rows[name] = {"shape": [b, h, t, d], "causal": bool(causal), "kernel": "attn_fwd_sw_kernel<128>" if causal
                      else "attn_fwd_pp_kernel<128> (the non-causal forward)",
                      "workgroups": b * h * (t // (256 if causal else 128)),
                      "us": sec * 1e6, "tflops": fl / sec / 1e12, "frac_bf16_peak": fl / sec / 1e12 / PEAK_BF16_TFLOPS}
        del q, k, v, o, lse
    return rows


def _rmsnorm_sets(rows, dim, sets, seed=0):
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    w = (1 + 0.1 * torch.randn(dim, device=dev, generator=g)).to(torch.bfloat16)
    bufs = []
    for _ in range(sets):
        x = torch.randn(rows, dim, device=dev, generator=g).to(torch.bfloat16)
        r = torch.randn(rows, dim, device=dev, generator=g).to(torch.bfloat16)
        bufs.append((x, r, torch.empty_like(x), torch.empty_like(x)))
    return w, bufs


def _graph_time(launch_all, iters, warmup, per):
    """Seconds per launch of `launch_all` (which enqueues `per` launches) replayed from a captured graph."""
    import torch

    launch_all()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch_all()
    t = _events_time(graph.replay, iters, warmup) / per
    del graph
    return t


def bench_stream_ceilings(nbytes: int = 1 << 30, iters: int = 10):
    """What this part's HBM streams reach at `nbytes` (1 GiB, far past the 256 MB Infinity Cache):
    read-only (ferrite_hip_stream_read), write-only (ferrite_hip_stream_fill) and the two-buffer
    copy of add+RMSNorm's access pattern (ferrite_hip_stream_copy2, half reads and half writes),
    each the best over a few persistent-grid sizes. The copy's rate is the ceiling of a kernel that
    reads and writes equal byte counts, as add+RMSNorm does."""
    import torch

    from ferrite import _hip

    lib, st = _hip.lib(), torch.cuda.current_stream().cuda_stream
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0").random_(0, 255)
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
    sink = torch.empty(4096, dtype=torch.int32, device="cuda:0")
    half = nbytes // 2
    read, fill = {}, {}
    for blocks in (256, 512, 1024, 2048):
        t = _events_time(lambda: _hip.check(lib.ferrite_hip_stream_read(src.data_ptr(), nbytes, sink.data_ptr(),
                                                                        blocks, st), "stream_read"), iters, 2)
        read[blocks] = nbytes / t / 1e9
        t = _events_time(lambda: _hip.check(lib.ferrite_hip_stream_fill(dst.data_ptr(), nbytes, 0x3F803F80, blocks,
                                                                        st), "stream_fill"), iters, 2)
        fill[blocks] = nbytes / t / 1e9
    # copy2 moves `nbytes` in all: two buffers of nbytes / 4 read, two written
    t = _events_time(lambda: _hip.check(lib.ferrite_hip_stream_copy2(src.data_ptr(), src.data_ptr() + half // 2,
                                                                     dst.data_ptr(), dst.data_ptr() + half // 2,
                                                                     half // 2, st), "stream_copy2"), iters, 2)
    copy = nbytes / t / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "read_gbs": max(read.values()), "write_gbs": max(fill.values()),
            "copy_read_plus_write_gbs": copy, "read_gbs_by_blocks": read, "write_gbs_by_blocks": fill,
            "copy_frac_of_peak": copy / PEAK_HBM_GBS}


def bench_mfma_ceiling(iters_per_launch: int = 4096, launches: int = 10):
    """What this part's matrix pipes sustain on bf16: ferrite_hip_mfma_ceiling (every wave streams
    independent v_mfma_f32_32x32x16_bf16 on register operands, no memory traffic) at one and two
    waves per SIMD and one and two workgroups per CU, each launch ~1 ms, after the bench's
    clock settling; the best rate is the ceiling of an MFMA-bound kernel on this part, as the
    stream kernels give the HBM one."""
    import torch

    from ferrite import _hip

    lib, st = _hip.lib(), torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.empty(2 * cus * 8, dtype=torch.float32, device="cuda:0")
    rates = {}
    for waves in (4, 8):
        for per_cu in (1, 2):
            blocks = per_cu * cus
            run = lambda: _hip.check(lib.ferrite_hip_mfma_ceiling(sink.data_ptr(), blocks, waves,  # noqa: E731
                                                                   iters_per_launch, st), "mfma_ceiling")
            _settle(run, 0.1)
            t = _events_time(run, launches, 1)
            rates[f"waves{waves}_x{per_cu}"] = blocks * waves * iters_per_launch * 8 * 32768 / t / 1e12
    best = max(rates.values())
    return {"bf16_tflops": best, "frac_of_spec_peak": best / PEAK_BF16_TFLOPS, "by_config": rates,
            "flops_per_launch_per_wave": iters_per_launch * 8 * 32768}


def bench_rmsnorm(rows, dim, steps, warmup, sets=24):
    """add+RMSNorm over `sets` rotating buffer sets (24 x 33.5 MB = 805 MB > the 256 MB MALL),
    launched through a captured HIP graph so host launch cost does not pace the ~7 us kernels.

    Beside it, copies of the same access pattern as references: the library's non-temporal
    two-buffer copy (ferrite_hip_stream_copy2: x -> h and r -> y, same bytes, same rotation and
    replay) and torch's copy, both at the bench size, and both kernels again at 16x the size (537 MB
    per launch, 3 sets), where the per-launch ramp no longer counts. `ratio_to_best_copy` is the
    kernel's rate over the fastest of those copies (a reference-copy ratio, not a ceiling: the
    kernel can beat a copy of its own bytes). The ceilings of this part's streams are measured by
    bench_stream_ceilings."""
    import torch

    from ferrite import _hip

    lib = _hip.lib()
    nbytes = 4 * rows * dim * 2 + dim * 2  # read x, r, w; write h, y
    copy_bytes = 4 * rows * dim * 2

    def norm_all(w, bufs, n):
        st = torch.cuda.current_stream().cuda_stream
        for x, r, hh, y in bufs:
            _hip.check(lib.ferrite_hip_add_rmsnorm(x.data_ptr(), r.data_ptr(), w.data_ptr(), hh.data_ptr(), y.data_ptr(),
                                                   n, dim, _hip.BF16, _hip.BF16, 1e-6, st), "add_rmsnorm")

    def copy_all(bufs, n):
        st = torch.cuda.current_stream().cuda_stream
        for x, r, hh, y in bufs:
            _hip.check(lib.ferrite_hip_stream_copy2(x.data_ptr(), r.data_ptr(), hh.data_ptr(), y.data_ptr(),
                                                    n * dim * 2, st), "stream_copy2")

    w, bufs = _rmsnorm_sets(rows, dim, sets)
    t = _graph_time(lambda: norm_all(w, bufs, rows), max(steps, 10), warmup, sets)
    t_eager = _events_time(lambda: norm_all(w, bufs, rows), max(steps // 2, 5), 2) / sets
    t_copy = _graph_time(lambda: copy_all(bufs, rows), max(steps, 10), warmup, sets)

    def torch_copy_all():
        for x, r, hh, y in bufs:
            hh.copy_(x)
            y.copy_(r)

    t_tcopy = _graph_time(torch_copy_all, max(steps, 10), warmup, sets)
    del bufs
    big_rows, big_sets = 16 * rows, 3
    w2, big = _rmsnorm_sets(big_rows, dim, big_sets, seed=1)
    t_big = _graph_time(lambda: norm_all(w2, big, big_rows), 10, 2, big_sets)
    t_big_copy = _graph_time(lambda: copy_all(big, big_rows), 10, 2, big_sets)
    del big
    torch.cuda.empty_cache()
    big_bytes, big_copy_bytes = 4 * big_rows * dim * 2 + dim * 2, 4 * big_rows * dim * 2
    same = copy_bytes / t_copy / 1e9
    torch_same = copy_bytes / t_tcopy / 1e9
    best_copy = max(same, torch_same, big_copy_bytes / t_big_copy / 1e9)
    gbs = nbytes / t / 1e9
    return {"shape": [rows, dim], "us": t * 1e6, "gbs": gbs, "bytes": nbytes,
            "frac_hbm": gbs / PEAK_HBM_GBS, "buffer_sets": sets, "eager_us": t_eager * 1e6,
            "stream_copy_same_bytes_us": t_copy * 1e6, "stream_copy_same_bytes_gbs": same,
            "torch_copy_same_bytes_us": t_tcopy * 1e6, "torch_copy_same_bytes_gbs": torch_same,
            "ratio_to_copy_same_bytes": gbs / same,
            "x16_size": {"shape": [big_rows, dim], "add_rmsnorm_us": t_big * 1e6,
                         "add_rmsnorm_gbs": big_bytes / t_big / 1e9, "stream_copy_us": t_big_copy * 1e6,
                         "stream_copy_gbs": big_copy_bytes / t_big_copy / 1e9},
            "best_copy_gbs": best_copy, "ratio_to_best_copy": gbs / best_copy}


def bench_matmul(steps, warmup):
    import torch

    from ferrite import _hip

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(3)
    out = {}
    # f32 first: right after a burst of bf16 4096^3 products the shader clock is still low
    # (1000^3 f32 then reads ~40 us instead of ~30, torch's ~29 instead of ~25), so the
    # second shape would be timed at whatever clock the first left behind. Each shape times
    # the library and torch alternately, three rounds, and keeps the median of each.
    for name, n, dt, code in (("f32_1000", 1000, torch.float32, _hip.F32), ("bf16_4096", 4096, torch.bfloat16, _hip.BF16)):
        a = (torch.rand(n, n, device=dev, generator=g) * 2 - 1).to(dt)
        bm = (torch.rand(n, n, device=dev, generator=g) * 2 - 1).to(dt)
        c = torch.empty(n, n, device=dev, dtype=dt)
        lib, st = _hip.lib(), _hip.stream_of(a)
        # what ferrite.kernels.matmul runs: the workspace from the size query, allocated once
        ws_bytes = lib.ferrite_hip_matmul_workspace(n, n, n, code)
        ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)

        def mm():
            _hip.check(lib.ferrite_hip_matmul_ex(a.data_ptr(), bm.data_ptr(), c.data_ptr(), n, n, n, 0, 0, code, code,
                                                 ws.data_ptr(), ws_bytes, st), "mm")

        ours, theirs = [], []
        for _ in range(3):
            ours.append(_events_time(mm, steps, warmup))
            theirs.append(_events_time(lambda: torch.matmul(a, bm), steps, warmup))
        t, t_torch = sorted(ours)[1], sorted(theirs)[1]
        peak = PEAK_BF16_TFLOPS if dt == torch.bfloat16 else PEAK_FP32_TFLOPS
        out[name] = {"us": t * 1e6, "tflops": 2 * n**3 / t / 1e12, "frac_peak": 2 * n**3 / t / 1e12 / peak,
                     "torch_matmul_us": t_torch * 1e6, "workspace_bytes": ws_bytes}
    return out


def bench_gpt_train(steps, warmup, linear_routes=("pallas", "xla"), modes=("graph", "eager")):
    """One GPT train step (forward + backward + AdamW) of BASELINE config 5: 12 layers, d_model 768,
    12 heads of 64, MLP 3072, vocab 32768, seq 1024, batch 8, bf16 parameters, tokens U[0, vocab).
    Attention, norms, loss, head layout and AdamW run on the HIP kernels; the linear layers on the
    HIP matmul ("pallas") or on torch's GEMM ("xla"). "graph" replays the step from a captured HIP
    graph, "eager" launches it from Python. FLOPs are the reference's analytic count
    (gpt.py:155-163)."""
    import torch

    from ferrite.model.gpt import GPTConfig, flops_per_token, init_params, param_count
    from ferrite.model.train import TrainConfig, adamw_init, build_train_step

    dev = torch.device("cuda:0")
    b = 8
    base = GPTConfig(vocab_size=32768, seq_len=1024, d_model=768, n_head=12, n_layer=12, d_ff=3072)
    g = torch.Generator().manual_seed(11)
    x = torch.randint(0, base.vocab_size, (b, base.seq_len), generator=g).to(dev)
    y = torch.randint(0, base.vocab_size, (b, base.seq_len), generator=g).to(dev)
    out = {}
    for route in linear_routes:
        for mode in modes:
            cfg = base.replace(linear=route)
            params = init_params(0, cfg, device=dev, param_dtype=torch.bfloat16)
            n_nonembed = param_count(params) - params["tok_emb"].numel() - params["pos_emb"].numel()
            flops = 3 * flops_per_token(cfg, n_nonembed)["total"] * b * cfg.seq_len
            opt = adamw_init(params)
            step = build_train_step(cfg, TrainConfig(steps=1000, warmup=10, lr=3e-4), graph=mode == "graph")
            losses = []

            def one():
                nonlocal params, opt
                params, opt, loss, _ = step(params, opt, x, y)
                losses.append(loss)

            t = _events_time(one, steps, max(warmup, 3))
            out[f"linear_{route}_{mode}"] = {
                "ms_per_step": t * 1e3, "tokens_per_s": b * cfg.seq_len / t, "tflops": flops / t / 1e12,
                "mfu_bf16": flops / t / 1e12 / PEAK_BF16_TFLOPS, "train_flops_per_step": flops,
                "params": param_count(params), "params_nonembed": n_nonembed,
                "loss_first": float(losses[0]), "loss_last": float(losses[-1]),
            }
            if hasattr(step, "close"):
                step.close()
            del params, opt, step, losses
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
    return out


def bench_decode_attention(iters=20):
    """Decode attention over a full static cache: B=8, H=32, max_len=8192, D=128 bf16, every
    sequence at its last position. HBM-bound: each call reads all keys and values once
    (8*32*8192*128*2*2 = 1.07 GB) and writes one row per head."""
    import torch

    from ferrite.kernels.decode_attention import decode_attention

    dev = torch.device("cuda:0")
    b, h, L, d = 8, 32, 8192, 128
    g = torch.Generator(device=dev).manual_seed(21)
    q, kn, vn = (torch.randn(b, h, d, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    kc = torch.randn(b, h, L, d, device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn(b, h, L, d, device=dev, generator=g).to(torch.bfloat16)
    pos = torch.full((b,), L - 1, dtype=torch.int32, device=dev)
    fn = lambda: decode_attention(q, kn, vn, kc, vc, pos)  # noqa: E731
    _settle(fn, 0.1)
    t = _events_time(fn, iters, 3)
    nbytes = 2 * b * h * L * d * 2 + 3 * b * h * d * 2 + 2 * b * h * d * 2
    return {"shape": [b, h, L, d], "us": t * 1e6, "gbs": nbytes / t / 1e9, "bytes": nbytes,
            "frac_hbm": nbytes / t / 1e9 / PEAK_HBM_GBS}


def bench_serving(new_tokens=128, prompt_len=100, batches=(1, 8, 32)):
    """The reference's serving benchmark (benchmarks/bench_serve.py): GPT seq 512, d_model 512,
    4 layers, 4 heads, d_ff 2048, bf16, random init; prompts of 100 tokens, 128 new tokens,
    greedy. Prefill and decode replay captured HIP graphs; decode attention runs on the HIP
    kernel ("pallas") or on torch math ("xla", the reference's XLA decode)."""
    import numpy as np
    import torch

    from ferrite.model.gpt import GPTConfig, init_params
    from ferrite.serving.engine import Engine, ServeConfig

    dev = torch.device("cuda:0")
    cfg = GPTConfig(seq_len=512, d_model=512, n_head=4, n_layer=4, d_ff=2048)
    params = init_params(0, cfg, device=dev)
    rng = np.random.default_rng(0)
    rows = []
    for batch in batches:
        for kernels in ("pallas", "xla"):
            eng = Engine(params, cfg, ServeConfig(batch=batch, max_len=cfg.seq_len, buckets=(64, 128, 256),
                                                  decode_kernels=kernels))
            prompts = [list(rng.integers(1, 256, size=prompt_len)) for _ in range(batch)]
            eng.generate(prompts, 4)
            _, stats = eng.generate(prompts, new_tokens)
            rows.append({"batch": batch, "decode_kernels": kernels, "prompt_len": prompt_len, "new_tokens": new_tokens,
                         **{k: round(v, 4) if isinstance(v, float) else v for k, v in stats.items()}})
            eng.close()
            del eng
    return rows


def bench_copy(nbytes: int = 256 << 20, iters: int = 5):
    """A plain device-to-device copy of `nbytes`: reads and writes exactly nbytes, so FETCH_SIZE and
    WRITE_SIZE of its dispatch calibrate the byte counters; also a ceiling for streaming kernels."""
    import torch

    src = torch.ones(nbytes // 4, device="cuda:0")
    dst = torch.empty_like(src)
    t = _events_time(lambda: dst.copy_(src), iters, 2)
    return {"bytes_each_way": nbytes, "us": t * 1e6, "gbs_read_plus_write": 2 * nbytes / t / 1e9}


def _blas_threads() -> int:
    try:
        import threadpoolctl

        info = [d for d in threadpoolctl.threadpool_info() if d.get("user_api") == "blas"]
        if info:
            return int(info[0]["num_threads"])
    except Exception:  # threadpoolctl missing or unreadable: fall back to the affinity mask
        pass
    return len(os.sched_getaffinity(0))


def _time_until(fn, budget_s: float, unit: int = 1) -> tuple[int, float]:
    """Call fn() after one untimed call until budget_s has passed and the count is a multiple of
    `unit`; returns (calls, seconds)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s and n % unit == 0:
            return n, el


def cpu_baseline(budget_s: float = 12.0):
    """The oracle's restatement of the reference's impl='xla' path (numpy f32 on this host's cores)
    on bounded samples of each BASELINE workload, reported in each kernel's own unit.

    Headline: the materialised f32 causal attention forward (oracle.attention.forward) over whole
    passes of the 64 (b, h) heads of 4x16x2048x128, TFLOP/s. Legs: add+RMSNorm at [4096, 1024]
    (oracle.rmsnorm.add_rmsnorm, f32 statistics, outputs rounded to bf16; GB/s of the bf16 bytes
    the kernel moves), and the matmul reference (f32 accumulation) at 4096^3 on bf16 values and
    at 1000^3 f32, TFLOP/s."""
    import numpy as np

    from oracle import attention as oatt
    from oracle import matmul as omm
    from oracle import rmsnorm as orms
    from oracle.bf16 import round_bf16

    blas = _blas_threads()
    b, h, t, d = 4, 16, 2048, 128
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, 1, t, d)).astype(np.float32) for _ in range(3))
    n, el = _time_until(lambda: oatt.forward(q, k, v, causal=True, dtype=np.float32), budget_s, unit=b * h)
    flops_head = 4 * t * t * d * 0.5
    out = {"value": round(flops_head * n / el / 1e12, 5), "unit": "TFLOP/s", "cores": blas, "kind": "port",
           "sample": f"{n // (b * h)} full passes over the {b * h} (b,h) heads of the 4x16x2048x128 causal forward "
                     f"({n} heads), oracle.attention.forward in numpy float32 (BLAS on {blas} threads), {el:.1f} s",
           "threads_env": os.environ.get("OMP_NUM_THREADS")}

    legs = {}
    rows, dim = 4096, 1024
    x = round_bf16(rng.standard_normal((rows, dim)).astype(np.float32))
    r = round_bf16(rng.standard_normal((rows, dim)).astype(np.float32))
    w = round_bf16((1 + 0.1 * rng.standard_normal(dim)).astype(np.float32))
    n, el = _time_until(lambda: orms.add_rmsnorm(x, w, r, out_bf16=True), budget_s / 3)
    nbytes = 4 * rows * dim * 2 + dim * 2
    legs["add_rmsnorm"] = {"value": round(nbytes * n / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                           "sample": f"{n} calls of oracle.rmsnorm.add_rmsnorm on [4096, 1024] (numpy elementwise, "
                                     f"one thread), {el:.1f} s; bytes counted as the bf16 kernel's 33,556,480"}
    for name, size, bf in (("matmul_bf16_4096", 4096, True), ("matmul_f32_1000", 1000, False)):
        a_ = rng.uniform(-1, 1, (size, size)).astype(np.float32)
        b_ = rng.uniform(-1, 1, (size, size)).astype(np.float32)
        if bf:
            a_, b_ = round_bf16(a_), round_bf16(b_)
        n, el = _time_until(lambda: omm.reference(a_, b_, out_bf16=bf, acc=np.float32), budget_s / 4)
        legs[name] = {"value": round(2 * size**3 * n / el / 1e12, 5), "unit": "TFLOP/s", "cores": blas,
                      "kind": "port",
                      "sample": f"{n} products of oracle.matmul.reference {size}^3 in numpy float32 "
                                f"({'bf16-valued inputs, output rounded to bf16' if bf else 'f32'}; BLAS on {blas} "
                                f"threads), {el:.1f} s"}
    out["legs"] = legs
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["attn", "rmsnorm", "matmul", "gpt", "serve", "all"], default="all")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (the HBM byte-counter calibration for rocprofv3 --pmc)")
    a = ap.parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (single-GPU tier); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from ferrite import _hip, platform

    _hip.lib()
    torch.cuda.synchronize()
    kernels = {}
    if a.calibrate_copy:
        kernels["copy_256MiB"] = bench_copy()
    if a.only in ("attn", "all"):
        kernels["attention"] = bench_attention(4, 16, 2048, 128, a.steps, a.warmup)
        kernels["attention_long_context"] = bench_attention(1, 8, 8192, 64, max(a.steps // 2, 3), 2, seed=27)
        kernels["attention_fwd_parts"] = bench_attention_fwd_parts(max(a.steps // 2, 5), 2)
        # Head dim 256 (the reference's tests run it), at the headline's FLOPs: the forward and dQ on
        # the pipelined four-wave kernels, dK/dV in one pass, four roles per 32-key block.
        kernels["attention_d256"] = bench_attention(4, 8, 2048, 256, max(a.steps // 5, 3), 2, seed=31)
        # The bf16 rate a pure MFMA stream sustains on this part, and each attention line against it.
        ceil = bench_mfma_ceiling()
        kernels["mfma_ceiling"] = ceil
        for key in ("attention", "attention_long_context", "attention_d256"):
            r = kernels[key]
            r["fwd_frac_of_measured_mfma_ceiling"] = r["fwd_tflops"] / ceil["bf16_tflops"]
            r["bwd_frac_of_measured_mfma_ceiling"] = r["bwd_tflops"] / ceil["bf16_tflops"]
    if a.only in ("rmsnorm", "all"):
        kernels["add_rmsnorm"] = bench_rmsnorm(4096, 1024, a.steps, a.warmup)
        ceil = bench_stream_ceilings()
        kernels["hbm_stream_ceilings"] = ceil
        r = kernels["add_rmsnorm"]
        # equal reads and writes: the copy's rate is this kernel's ceiling on this part
        r["frac_of_measured_ceiling"] = r["gbs"] / ceil["copy_read_plus_write_gbs"]
        r["x16_size"]["frac_of_measured_ceiling"] = r["x16_size"]["add_rmsnorm_gbs"] / ceil["copy_read_plus_write_gbs"]
    if a.only in ("matmul", "all"):
        kernels["matmul"] = bench_matmul(max(a.steps // 2, 3), 2)
    if a.only in ("gpt", "all"):
        kernels["gpt_train_step"] = bench_gpt_train(max(a.steps // 2, 3), 2)
    if a.only in ("serve", "all"):
        kernels["decode_attention"] = bench_decode_attention()
        kernels["serving"] = bench_serving()

    att = kernels.get("attention")
    if att is not None:
        value = att["fwd_tflops"]
        ms = att["fwd_us"] / 1e3
        roof = _roofline("attn_fwd", att["flops_fwd"], att["bytes_fwd"], att["fwd_us"] * 1e-6,
                         traffic=_traffic("attn_fwd"))
    else:  # partial runs report the first kernel measured
        first = next(iter(kernels.values()))
        value, ms, roof = first.get("gbs", first.get("tflops", 0.0)), first.get("us", 0.0) / 1e3, None
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "causal flash attention forward, q,k,v bf16 [B=4,H=16,T=2048,d=128] ~ N(0,1), "
                               "scale 1/sqrt(128); step = one forward over the batch",
                   "global_batch": 4, "seq_len": 2048, "heads": 16, "head_dim": 128, "parallelism": "none (1 GPU)"},
        "roofline": roof,
        "cpu_baseline": None if a.no_cpu_baseline else cpu_baseline(),
        "kernels": kernels,
        "platform": platform.describe(),
    }
    if "add_rmsnorm" in kernels:
        r = kernels["add_rmsnorm"]
        line["add_rmsnorm_roofline"] = _roofline("add_rmsnorm", 5 * r["shape"][0] * r["shape"][1], r["bytes"],
                                                 r["us"] * 1e-6, traffic=_traffic("add_rmsnorm"))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
