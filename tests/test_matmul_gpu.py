"""GPU parity of the blocked MFMA matmul against the oracle.

Reference tests mirrored: tests/test_matmul.py:13-41. bf16
4096^3 (U(-1,1)) and ragged f32 1000^3 (relative error <= 1e-5). The bf16
output bar of BASELINE (2e-2 max-abs against the f32 product) is below the
bf16 rounding of outputs of magnitude ~100, so the bf16 product is held to one
bf16 ulp of the rounded exact product and a relative error bar instead.
"""

import numpy as np
import pytest
import torch

from ferrite import _hip
from ferrite.kernels import matmul
from oracle import matmul as omm
from tests._util import bf16_ulp, normal, rel_fro, to_dev, to_np, uniform

pytestmark = pytest.mark.gpu


def test_baseline_bf16_4096(dev):
    a, b = uniform(3, (4096, 4096), "bf16"), uniform(4, (4096, 4096), "bf16")
    out = matmul(to_dev(a, "bf16", dev), to_dev(b, "bf16", dev))
    assert out.dtype == torch.bfloat16 and out.shape == (4096, 4096)
    exact = omm.reference(a, b)  # f64 accumulation, f32 result
    g = to_np(out).astype(np.float64)
    # One bf16 ulp of the exact product plus the f32 accumulation error bound (2^-20 sum|a||b|,
    # which matters only where the product cancels to near zero).
    absab = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    assert np.all(np.abs(g - exact) <= bf16_ulp(exact) + 2.0**-20 * absab)
    assert np.mean(g != omm.reference(a, b, out_bf16=True)) < 0.01  # almost all equal bf16(exact)
    assert rel_fro(g, exact) < 4e-3


def test_ragged_f32_1000(dev):
    a, b = uniform(5, (1000, 1000)), uniform(6, (1000, 1000))
    out = to_np(matmul(to_dev(a, "f32", dev), to_dev(b, "f32", dev)))
    exact = omm.reference(a, b)
    rel = np.max(np.abs(out.astype(np.float64) - exact)) / np.max(np.abs(exact))
    assert rel <= 1e-5, rel


@pytest.mark.parametrize("dtype,atol", [("f32", 1e-3), ("bf16", 0.5)])
def test_matches_reference_aligned(dev, dtype, atol):
    """tests/test_matmul.py:13-20."""
    x, y = normal(7, (256, 384), dtype), normal(8, (384, 512), dtype)
    out = matmul(to_dev(x, dtype, dev), to_dev(y, dtype, dev), block_m=128, block_n=256, block_k=128)
    assert out.shape == (256, 512)
    np.testing.assert_allclose(to_np(out), omm.reference(x, y, out_bf16=dtype == "bf16"), atol=atol, rtol=1e-2)


def test_ragged_shapes_are_padded_exactly(dev):
    """tests/test_matmul.py:23-27, plus exactness on integer-valued inputs (every f32 sum is exact,
    so any accumulation order must reproduce the zero-padded product bit for bit)."""
    x, y = normal(9, (77, 130)), normal(10, (130, 203))
    out = matmul(to_dev(x, "f32", dev), to_dev(y, "f32", dev), block_m=64, block_n=128, block_k=128)
    np.testing.assert_allclose(to_np(out), omm.reference(x, y), atol=1e-3, rtol=1e-3)
    rng = np.random.default_rng(11)
    xi = rng.integers(-8, 9, (77, 130)).astype(np.float32)
    yi = rng.integers(-8, 9, (130, 203)).astype(np.float32)
    exact = omm.blocked_padded(xi, yi, bm=64, bn=128, bk=128)
    for dt in ("f32", "bf16"):
        got = to_np(matmul(to_dev(xi, dt, dev), to_dev(yi, dt, dev), out_dtype=torch.float32))
        np.testing.assert_array_equal(got, exact)


def test_f32_output_from_bf16_inputs(dev):
    """tests/test_matmul.py:30-35."""
    x, y = normal(12, (128, 256), "bf16"), normal(13, (256, 128), "bf16")
    out = matmul(to_dev(x, "bf16", dev), to_dev(y, "bf16", dev), out_dtype=torch.float32)
    assert out.dtype == torch.float32
    np.testing.assert_allclose(to_np(out), omm.reference(x, y), atol=1e-2, rtol=1e-2)
    out2 = matmul(to_dev(x, "bf16", dev), to_dev(y, "bf16", dev), out_dtype="float32")
    assert out2.dtype == torch.float32


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 7, 3), (33, 17, 65), (300, 1000, 4100), (513, 64, 257), (64, 4096, 8)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_edge_shapes(dev, m, k, n, dtype):
    x, y = uniform(14, (m, k), dtype), uniform(15, (k, n), dtype)
    out = to_np(matmul(to_dev(x, dtype, dev), to_dev(y, dtype, dev), out_dtype=torch.float32))
    exact = omm.reference(x, y)
    assert np.max(np.abs(out - exact)) <= 1e-5 * max(1.0, np.max(np.abs(exact))) * (1 + k / 64)


def test_bf16_output_from_f32_inputs(dev):
    x, y = uniform(16, (200, 300)), uniform(17, (300, 100))
    out = matmul(to_dev(x, "f32", dev), to_dev(y, "f32", dev), out_dtype=torch.bfloat16)
    exact = omm.reference(x, y)
    assert np.all(np.abs(to_np(out) - exact) <= bf16_ulp(exact))


def test_gradients(dev):
    """The VJP (matmul.py:99-104): dX = G Y^T, dY = X^T G through the same kernel."""
    x, y, g = normal(18, (64, 96)), normal(19, (96, 80)), normal(20, (64, 80))
    xt, yt = to_dev(x, "f32", dev).requires_grad_(), to_dev(y, "f32", dev).requires_grad_()
    (matmul(xt, yt) * to_dev(g, "f32", dev)).sum().backward()
    np.testing.assert_allclose(to_np(xt.grad), g.astype(np.float64) @ y.T, atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(to_np(yt.grad), x.T.astype(np.float64) @ g, atol=1e-4, rtol=1e-4)


def test_every_element_written_and_deterministic(dev):
    m, k, n = 1000, 520, 777
    x, y = uniform(21, (m, k), "bf16"), uniform(22, (k, n), "bf16")
    xt, yt = to_dev(x, "bf16", dev), to_dev(y, "bf16", dev)
    outs = []
    for _ in range(2):
        o = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        _hip.check(_hip.lib().ferrite_hip_matmul(xt.data_ptr(), yt.data_ptr(), o.data_ptr(), m, n, k, _hip.BF16,
                                                 _hip.F32, _hip.stream_of(xt)), "matmul")
        torch.cuda.synchronize()
        assert not torch.isnan(o).any()
        outs.append(o.clone())
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("m,k,n", [
    (1000, 1000, 1000),  # 4 K slices in each workgroup (the BASELINE f32 shape)
    (1000, 1003, 999),   # the same, unaligned rows (N % 4 != 0)
    (512, 2048, 512),    # 4 slices per workgroup x 4 groups of workgroups, summed from the workspace
    (132, 2050, 67),     # groups of slices, unaligned rows and a ragged last slice
    (1400, 700, 1400),   # 2 slices per workgroup (4 would exceed two waves per SIMD)
    (300, 300, 300),     # 2 slices, K under 512
    (100, 100, 100),     # no split (K too short for 128-deep slices)
])
def test_f32_small_products_split_k(dev, m, k, n):
    """f32 products with few output tiles split K inside the workgroup (and, with very few
    tiles, across workgroups through the workspace). Every element is written (NaN-prefilled),
    the result is within 1e-5 of the f64 product relative to its largest magnitude, and two
    runs are bitwise equal (the slices are summed in a fixed order)."""
    x, y = uniform(31, (m, k), "f32"), uniform(32, (k, n), "f32")
    xt, yt = to_dev(x, "f32", dev), to_dev(y, "f32", dev)
    exact = x.astype(np.float64) @ y.astype(np.float64)
    lib = _hip.lib()
    ws_bytes = lib.ferrite_hip_matmul_workspace(m, n, k, _hip.F32)
    ws = torch.empty(max(ws_bytes, 16) // 4, dtype=torch.float32, device=dev)
    for out_code, tdt in ((_hip.F32, torch.float32), (_hip.BF16, torch.bfloat16)):
        outs = []
        for _ in range(2):
            o = torch.full((m, n), float("nan"), dtype=tdt, device=dev)
            _hip.check(lib.ferrite_hip_matmul_ex(xt.data_ptr(), yt.data_ptr(), o.data_ptr(), m, n, k, 0, 0, _hip.F32,
                                                 out_code, ws.data_ptr(), ws_bytes, _hip.stream_of(xt)), "matmul")
            torch.cuda.synchronize()
            outs.append(o.clone())
        got = to_np(outs[0]).astype(np.float64)
        assert not np.isnan(got).any()
        assert torch.equal(outs[0], outs[1])
        if tdt == torch.float32:
            assert np.max(np.abs(got - exact)) <= 1e-5 * np.max(np.abs(exact))
        else:
            assert np.all(np.abs(got - exact) <= bf16_ulp(exact) + 1e-5 * np.max(np.abs(exact)))


@pytest.mark.parametrize("m,k,n", [
    (2048, 1000, 2048),  # 256 tiles of 128 x 128: the pipelined loop on the large tiles, 16-byte rows
    (2100, 1003, 2050),  # the same with 4-byte loads (K and N not multiples of 4), ragged tiles
    (2048, 64, 2176),    # one pass of the loop (two k-steps)
])
def test_f32_large_products_pipelined(dev, m, k, n):
    """f32 products with a CU's worth of 128 x 128 tiles run the pipelined loop on those tiles:
    every element written (NaN-prefilled), within 1e-5 of the f64 product relative to its largest
    magnitude (bf16 output: one bf16 ulp more), and two runs bitwise equal."""
    x, y = uniform(41, (m, k), "f32"), uniform(42, (k, n), "f32")
    xt, yt = to_dev(x, "f32", dev), to_dev(y, "f32", dev)
    exact = x.astype(np.float64) @ y.astype(np.float64)
    lib = _hip.lib()
    assert lib.ferrite_hip_matmul_workspace(m, n, k, _hip.F32) == 0
    for out_code, tdt in ((_hip.F32, torch.float32), (_hip.BF16, torch.bfloat16)):
        outs = []
        for _ in range(2):
            o = torch.full((m, n), float("nan"), dtype=tdt, device=dev)
            _hip.check(lib.ferrite_hip_matmul_ex(xt.data_ptr(), yt.data_ptr(), o.data_ptr(), m, n, k, 0, 0, _hip.F32,
                                                 out_code, None, 0, _hip.stream_of(xt)), "matmul")
            torch.cuda.synchronize()
            outs.append(o.clone())
        got = to_np(outs[0]).astype(np.float64)
        assert not np.isnan(got).any()
        assert torch.equal(outs[0], outs[1])
        if tdt == torch.float32:
            assert np.max(np.abs(got - exact)) <= 1e-5 * np.max(np.abs(exact))
        else:
            assert np.all(np.abs(got - exact) <= bf16_ulp(exact) + 1e-5 * np.max(np.abs(exact)))


@pytest.mark.parametrize("m,k,n", [(300, 128, 264), (257, 192, 520), (1000, 512, 776), (64, 64, 8)])
def test_bf16_dma_path_tails(dev, m, k, n):
    """bf16 inputs with K a multiple of 64 and N a multiple of 8 take the DMA-fed kernel, whose
    tiles are 256 x 256: rows past M and columns past N must read as zeros and never be stored.
    Every output element is written (NaN-prefilled), f32 out matches the f64 product to the
    accumulation bar, bf16 out is within one bf16 ulp of the exact product."""
    x, y = uniform(23, (m, k), "bf16"), uniform(24, (k, n), "bf16")
    xt, yt = to_dev(x, "bf16", dev), to_dev(y, "bf16", dev)
    exact = omm.reference(x, y)
    for out_code, tdt in ((_hip.F32, torch.float32), (_hip.BF16, torch.bfloat16)):
        o = torch.full((m, n), float("nan"), dtype=tdt, device=dev)
        _hip.check(_hip.lib().ferrite_hip_matmul(xt.data_ptr(), yt.data_ptr(), o.data_ptr(), m, n, k, _hip.BF16,
                                                 out_code, _hip.stream_of(xt)), "matmul")
        torch.cuda.synchronize()
        got = to_np(o)
        assert not np.isnan(got).any()
        if tdt == torch.float32:
            assert np.max(np.abs(got - exact)) <= 1e-5 * max(1.0, np.max(np.abs(exact))) * (1 + k / 64)
        else:
            assert np.all(np.abs(got - exact) <= bf16_ulp(exact) + 2.0 ** -20 * np.abs(x).sum(1, keepdims=True) @ np.abs(y).max(0, keepdims=True))


_EXACT = {}


def _exact_case(m, n, k):
    """Seeded bf16 operands, their f64 product and the f32 accumulation bound (cached per shape)."""
    if (m, n, k) not in _EXACT:
        a = uniform(40 + m % 13, (m, k), "bf16")
        b = uniform(41 + n % 11, (k, n), "bf16")
        bound = 2.0**-20 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)) + 1e-30
        _EXACT.clear()
        _EXACT[(m, n, k)] = (a, b, omm.reference(a, b), bound)
    return _EXACT[(m, n, k)]


def _mm_ex(xs, ys, m, n, k, x_t, y_t, out_dtype, workspace=True):
    """ferrite_hip_matmul_ex through the C ABI on NaN-prefilled output."""
    lib = _hip.lib()
    out = torch.full((m, n), float("nan"), dtype=out_dtype, device=xs.device)
    ws_bytes = lib.ferrite_hip_matmul_workspace(m, n, k, _hip.BF16) if workspace else 0
    ws = torch.full(((ws_bytes + 3) // 4,), float("nan"), device=xs.device) if ws_bytes > 0 else None
    rc = lib.ferrite_hip_matmul_ex(xs.data_ptr(), ys.data_ptr(), out.data_ptr(), m, n, k, int(x_t), int(y_t), _hip.BF16,
                                   _hip.dtype_code(out_dtype), _hip.ptr(ws), max(ws_bytes, 0), _hip.stream_of(xs))
    _hip.check(rc, "matmul_ex")
    torch.cuda.synchronize()
    return out, ws_bytes


@pytest.mark.parametrize("m,n,k", [
    (768, 3072, 8192),   # a GPT weight gradient: 36 tiles, K split 8 ways
    (768, 768, 4096),    # 9 tiles, K split 8 ways (512 deep)
    (520, 264, 1024),    # ragged tile edges, K split
    (1024, 2304, 768),   # 36 tiles but K too short to split
    (8192, 768, 3072),   # 96 tiles: 128-row tiles (k-contiguous x), else long K split 2 ways
    (8192, 768, 512),    # 128-row tiles (k-contiguous x), else no split
    (8192, 2304, 768),   # 288 256-row tiles: 576 128-row ones with a k-contiguous x
    (2000, 2056, 320),   # 128-row tiles with ragged row and column edges
])
@pytest.mark.parametrize("x_t,y_t", [(False, False), (True, False), (False, True), (True, True)])
def test_transposed_operands_and_k_split(dev, m, n, k, x_t, y_t):
    """out = op(x) @ op(y) with x and/or y read transposed in place, against the f64 product of the
    same bf16 values: f32 output within the f32 accumulation bound, bf16 output within one bf16 ulp
    of the exact product plus that bound. Every element is written, reruns are bitwise equal,
    and the split and unsplit kernels agree to the f32 bound."""
    a, b, exact, bound = _exact_case(m, n, k)
    xs = to_dev(a.T.copy() if x_t else a, "bf16", dev)
    ys = to_dev(b.T.copy() if y_t else b, "bf16", dev)
    o32, ws_bytes = _mm_ex(xs, ys, m, n, k, x_t, y_t, torch.float32)
    assert not torch.isnan(o32).any()
    assert np.all(np.abs(to_np(o32).astype(np.float64) - exact) <= bound)
    again, _ = _mm_ex(xs, ys, m, n, k, x_t, y_t, torch.float32)
    assert torch.equal(o32, again)
    nosplit, _ = _mm_ex(xs, ys, m, n, k, x_t, y_t, torch.float32, workspace=False)
    assert np.all(np.abs(to_np(nosplit).astype(np.float64) - exact) <= bound)
    o16, _ = _mm_ex(xs, ys, m, n, k, x_t, y_t, torch.bfloat16)
    assert np.all(np.abs(to_np(o16).astype(np.float64) - exact) <= bf16_ulp(exact) + bound)
    if m * n <= 768 * 768 and k >= 4096:
        assert ws_bytes > 0  # the small-output shapes do split


def test_transposed_operand_rules(dev):
    """Transposed operands outside the DMA kernel's rule return an error; the Python wrapper
    transposes into a copy instead (the VJP then still matches)."""
    lib = _hip.lib()
    x = torch.zeros(64, 100, device=dev, dtype=torch.bfloat16)  # K = 100: not a multiple of 64
    y = torch.zeros(100, 64, device=dev, dtype=torch.bfloat16)
    out = torch.empty(64, 64, device=dev, dtype=torch.bfloat16)
    rc = lib.ferrite_hip_matmul_ex(x.data_ptr(), y.data_ptr(), out.data_ptr(), 64, 64, 100, 0, 1, _hip.BF16, _hip.BF16,
                                   None, 0, _hip.stream_of(x))
    assert rc == 1 and "transposed" in _hip.last_error()


@pytest.mark.parametrize("m,k,n", [(1024, 768, 2304), (1000, 136, 72)])
def test_vjp_reads_transposes_in_place(dev, m, k, n):
    """Gradients of matmul through autograd (dx = g y^T, dy = x^T g on the transposed-operand
    kernel, or on copies for shapes outside its rule) against f64 products of the same bf16 values,
    held to the bf16 output bar (one ulp plus the f32 accumulation bound)."""
    a, b, gg = normal(50, (m, k), "bf16"), normal(51, (k, n), "bf16"), normal(52, (m, n), "bf16")
    xt, yt = to_dev(a, "bf16", dev).requires_grad_(), to_dev(b, "bf16", dev).requires_grad_()
    matmul(xt, yt).backward(to_dev(gg, "bf16", dev))
    for got, ex, absb in ((xt.grad, gg.astype(np.float64) @ b.T.astype(np.float64),
                           np.abs(gg).astype(np.float64) @ np.abs(b.T).astype(np.float64)),
                          (yt.grad, a.T.astype(np.float64) @ gg.astype(np.float64),
                           np.abs(a.T).astype(np.float64) @ np.abs(gg).astype(np.float64))):
        g64 = to_np(got).astype(np.float64)
        assert np.all(np.abs(g64 - ex) <= bf16_ulp(ex) + 2.0**-20 * absb + 1e-30)


@pytest.mark.parametrize("x_t,y_t", [(False, False), (True, False), (False, True)])
def test_four_wave_tiles_match_eight_wave_tiles(dev, x_t, y_t):
    """An 8192 x 8192 output has four rounds of 256 x 256 tiles and runs on four waves per tile; a
    2048 x 8192 one (one round) on eight. Both accumulate every output over the same 64-deep k
    steps in the same order, so the first 2048 rows agree bitwise, with either operand read
    transposed in place; the whole product is also held to the bf16 bar on sampled rows against
    the f64 product of the same values."""
    k = 256
    a = normal(95, (8192, k), "bf16")
    b = normal(96, (k, 8192), "bf16")
    xs = to_dev(a.T.copy() if x_t else a, "bf16", dev)
    ys = to_dev(b.T.copy() if y_t else b, "bf16", dev)
    big, _ = _mm_ex(xs, ys, 8192, 8192, k, x_t, y_t, torch.bfloat16)
    x_top = xs[:, :2048].contiguous() if x_t else xs[:2048].contiguous()
    top, _ = _mm_ex(x_top, ys, 2048, 8192, k, x_t, y_t, torch.bfloat16)
    assert torch.equal(big[:2048], top)
    rows = np.arange(0, 8192, 97)
    exact = a[rows].astype(np.float64) @ b.astype(np.float64)
    absb = np.abs(a[rows]).astype(np.float64) @ np.abs(b).astype(np.float64)
    got = to_np(big)[rows].astype(np.float64)
    assert np.all(np.abs(got - exact) <= bf16_ulp(exact) + 2.0**-20 * absb + 1e-30)


def _ceiling_operands():
    """The bf16 operands every lane of ferrite_hip_mfma_ceiling builds, as A[32, 16] and B[16, 32]
    of v_mfma_f32_32x32x16_bf16 (lane l holds A[l % 32, 8 (l // 32) + e] and B[8 (l // 32) + e, l % 32])."""
    from oracle.bf16 import round_bf16

    A = np.zeros((32, 16)); B = np.zeros((16, 32))
    for lane in range(64):
        for e in range(8):
            h = ((lane * 8 + e + 1) * 2654435761) & 0xFFFFFFFF
            av = float(np.asarray(round_bf16(np.float32(((h >> 8) & 0xFFFF) * (1.0 / 65536.0) - 0.5))).reshape(-1)[0])
            bv = float(np.asarray(round_bf16(np.float32(((h >> 16) & 0xFF) * (1.0 / 256.0) - 0.5))).reshape(-1)[0])
            A[lane % 32, 8 * (lane // 32) + e] = av
            B[8 * (lane // 32) + e, lane % 32] = bv
    return A, B


@pytest.mark.parametrize("waves,blocks,iters", [(8, 256, 64), (4, 512, 16)])
def test_mfma_ceiling_runs_its_products(dev, waves, blocks, iters):
    """The MFMA ceiling bench.py times does the products it is credited with: lane 0 of every wave
    leaves the sum of its accumulators, iters x 8 x (rows 8 (r // 4) + r % 4 of column 0 of A B),
    in sink, the same in every wave."""
    lib = _hip.lib()
    sink = torch.full((blocks * waves,), float("nan"), device=dev)
    _hip.check(lib.ferrite_hip_mfma_ceiling(sink.data_ptr(), blocks, waves, iters, _hip.stream_of(sink)), "ceiling")
    torch.cuda.synchronize()
    got = to_np(sink)
    A, B = _ceiling_operands()
    D = A @ B
    rows = [8 * (r // 4) + (r % 4) for r in range(16)]
    want = iters * 8 * D[rows, 0].sum()
    assert np.all(got == got[0]), "every wave computes the same sum"
    assert abs(got[0] - want) <= 1e-4 * iters * 8 * np.abs(D[rows, 0]).sum() + 1e-6, (got[0], want)
