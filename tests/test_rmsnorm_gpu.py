"""GPU parity of the fused add+RMSNorm kernel against the oracle.

Reference tests mirrored: tests/test_rmsnorm.py:9-54 (forward shapes, fused
residual, gradients). Bars: h bit-exact in bf16; y within 2e-2 max-abs of the
exact (f64-statistics) result and within one bf16 ulp of the reference's own
f32-statistics rounding; f32 outputs within 1e-5.
"""

import numpy as np
import pytest
import torch

from ferrite import _hip
from ferrite.kernels import rmsnorm
from oracle import rmsnorm as orms
from oracle.bf16 import round_bf16
from tests._util import bf16_ulp, max_abs, normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _check_bf16(h, y, x, w, r, eps=1e-6):
    h_ref, y32 = orms.add_rmsnorm(x, w, r, eps=eps, out_bf16=True)
    _, y64 = orms.add_rmsnorm(x, w, r, eps=eps, acc=np.float64)
    np.testing.assert_array_equal(to_np(h).view(np.uint32), h_ref.view(np.uint32))
    yg = to_np(y)
    assert max_abs(yg, y64) <= 2e-2
    assert np.all(np.abs(yg.astype(np.float64) - y32) <= bf16_ulp(y32))
    return yg


def test_baseline_config_add_rmsnorm(dev):
    """BASELINE config: x, r bf16 [4096,1024] ~ N(0,1), w bf16 = 1 + 0.1 N(0,1), eps 1e-6."""
    x = normal(0, (4096, 1024), "bf16")
    r = normal(1, (4096, 1024), "bf16")
    w = normal(2, (1024,), "bf16", loc=1.0, scale=0.1)
    h, y = rmsnorm(to_dev(x, "bf16", dev), to_dev(w, "bf16", dev), residual=to_dev(r, "bf16", dev), eps=1e-6)
    assert h.dtype == y.dtype == torch.bfloat16
    _check_bf16(h, y, x, w, r)


@pytest.mark.parametrize("shape", [(4, 64, 256), (300, 384), (2, 8, 128)])
def test_forward_matches_reference(dev, shape):
    """tests/test_rmsnorm.py:9-14 (f32, atol = rtol = 1e-5)."""
    x = normal(3, shape)
    w = normal(4, shape[-1:], loc=1.0, scale=0.1)
    y = rmsnorm(to_dev(x, "f32", dev), to_dev(w, "f32", dev))
    np.testing.assert_allclose(to_np(y), orms.add_rmsnorm(x, w, acc=np.float64), atol=1e-5, rtol=1e-5)


def test_fused_residual_forward(dev):
    """tests/test_rmsnorm.py:17-25 (bf16 2x256x256, w = 1)."""
    x, r = normal(5, (2, 256, 256), "bf16"), normal(6, (2, 256, 256), "bf16")
    w = np.ones(256, np.float32)
    h, y = rmsnorm(to_dev(x, "bf16", dev), to_dev(w, "bf16", dev), residual=to_dev(r, "bf16", dev))
    _check_bf16(h.reshape(-1, 256), y.reshape(-1, 256), x.reshape(-1, 256), w, r.reshape(-1, 256))


@pytest.mark.parametrize("rows,dim", [(1, 1024), (3, 1024), (37, 100), (8, 8192), (5, 4096), (64, 2048), (16, 8)])
def test_shapes_and_paths(dev, rows, dim):
    """Vector path (dim % 8 == 0, dim <= 4096), generic path (other dims), odd row counts."""
    x, r = normal(7, (rows, dim), "bf16"), normal(8, (rows, dim), "bf16")
    w = normal(9, (dim,), "bf16", loc=1.0, scale=0.1)
    h, y = rmsnorm(to_dev(x, "bf16", dev), to_dev(w, "bf16", dev), residual=to_dev(r, "bf16", dev))
    _check_bf16(h, y, x, w, r)
    y2 = rmsnorm(to_dev(x, "bf16", dev), to_dev(w, "bf16", dev))
    y2_ref = round_bf16(orms.add_rmsnorm(x, w))
    assert np.all(np.abs(to_np(y2).astype(np.float64) - y2_ref) <= bf16_ulp(y2_ref))


def test_f32_weight_with_bf16_activations(dev):
    """The model's case (gpt.py:75, :108-109): f32 weight, bf16 x and residual."""
    x, r = normal(10, (256, 768), "bf16"), normal(11, (256, 768), "bf16")
    w = normal(12, (768,), "f32", loc=1.0, scale=0.1)
    h, y = rmsnorm(to_dev(x, "bf16", dev), to_dev(w, "f32", dev), residual=to_dev(r, "bf16", dev))
    _check_bf16(h, y, x, w, r)


def test_mixed_residual_dtype(dev):
    x = normal(13, (64, 256), "bf16")
    r = normal(14, (64, 256), "f32")
    w = np.ones(256, np.float32)
    h, y = rmsnorm(to_dev(x, "bf16", dev), to_dev(w, "f32", dev), residual=to_dev(r, "f32", dev))
    _check_bf16(h, y, x, w, r)


def test_gradients_match_reference(dev):
    """tests/test_rmsnorm.py:28-44: loss = sum(y * cot) + sum(h * cot[::-1]), f32, 1e-4."""
    x, r = normal(15, (64, 256)), normal(16, (64, 256))
    w = normal(17, (256,), loc=1.0, scale=0.1)
    cot = normal(18, (64, 256))
    xt, rt, wt = (to_dev(a, "f32", dev).requires_grad_() for a in (x, r, w))
    h, y = rmsnorm(xt, wt, residual=rt)
    c = to_dev(cot, "f32", dev)
    (torch.sum(y * c) + torch.sum(h * c.flip(0))).backward()
    hh = x + r
    dh, dw = orms.rmsnorm_bwd(hh, w, cot)
    dh = dh + cot[::-1]
    np.testing.assert_allclose(to_np(xt.grad), dh, atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(to_np(rt.grad), dh, atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(to_np(wt.grad), dw, atol=1e-4, rtol=1e-4)


def test_plain_gradient(dev):
    """tests/test_rmsnorm.py:47-54: loss = sum(tanh(rmsnorm(x, w))), 1e-5."""
    x = normal(19, (32, 128))
    w = np.ones(128, np.float32)
    xt, wt = to_dev(x, "f32", dev).requires_grad_(), to_dev(w, "f32", dev).requires_grad_()
    torch.sum(torch.tanh(rmsnorm(xt, wt))).backward()
    y = orms.add_rmsnorm(x, w, acc=np.float64)
    dx, dw = orms.rmsnorm_bwd(x, w, 1.0 - np.tanh(y) ** 2)
    np.testing.assert_allclose(to_np(xt.grad), dx, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(to_np(wt.grad), dw, atol=1e-5, rtol=1e-5)


def test_every_element_written_and_deterministic(dev):
    """NaN-prefilled outputs through the C ABI: every element is written; reruns are bitwise equal."""
    rows, dim = 1000, 1024
    x, r = normal(20, (rows, dim), "bf16"), normal(21, (rows, dim), "bf16")
    w = normal(22, (dim,), "bf16", loc=1.0, scale=0.1)
    xt, rt, wt = to_dev(x, "bf16", dev), to_dev(r, "bf16", dev), to_dev(w, "bf16", dev)
    outs = []
    for _ in range(2):
        h = torch.full_like(xt, float("nan"))
        y = torch.full_like(xt, float("nan"))
        rc = _hip.lib().ferrite_hip_add_rmsnorm(xt.data_ptr(), rt.data_ptr(), wt.data_ptr(), h.data_ptr(), y.data_ptr(),
                                                rows, dim, _hip.BF16, _hip.BF16, 1e-6, _hip.stream_of(xt))
        _hip.check(rc, "add_rmsnorm")
        torch.cuda.synchronize()
        assert not torch.isnan(h).any() and not torch.isnan(y).any()
        outs.append((h.clone(), y.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def _bwd_abi(h, w, dy, dd, dh_dtype, dim_slice=None):
    """Run ferrite_hip_rmsnorm_bwd on device tensors; NaN-prefilled outputs."""
    rows, dim = h.shape
    lib = _hip.lib()
    dh = torch.full((rows, dim), float("nan"), dtype=dh_dtype, device=h.device)
    dw = torch.full_like(w, float("nan"))
    ws = torch.full(((lib.ferrite_hip_rmsnorm_bwd_workspace(rows, dim) + 3) // 4,), float("nan"), device=h.device)
    rc = lib.ferrite_hip_rmsnorm_bwd(h.data_ptr(), w.data_ptr(), dy.data_ptr(), _hip.ptr(dd), dh.data_ptr(),
                                     dw.data_ptr(), ws.data_ptr(), rows, dim, _hip.dtype_code(h.dtype),
                                     _hip.dtype_code(w.dtype), _hip.dtype_code(dh_dtype), 1e-6, _hip.stream_of(h))
    _hip.check(rc, "rmsnorm_bwd")
    torch.cuda.synchronize()
    return dh, dw


@pytest.mark.parametrize("rows,dim,dtype,direct", [
    (8192, 768, "bf16", True),    # the GPT's residual stream: row pass, VPL 2
    (8192, 768, "bf16", False),
    (4096, 1024, "bf16", True),
    (333, 4096, "f32", True),     # VPL 8, ragged row count
    (77, 64, "f32", False),       # VPL 1 with idle lanes
    (50, 100, "f32", True),       # dim % 8 != 0: general row pass + column pass
    (19, 5000, "bf16", False),    # dim above the register path: general
    (3, 768, "bf16", True),       # fewer rows than waves
])
def test_bwd_kernel_matches_oracle(dev, rows, dim, dtype, direct):
    """dh and dweight of ferrite_hip_rmsnorm_bwd against the f64 analytic backward
    (rmsnorm.py:159-166, + the direct term of :148-153). f32: 1e-4 relative to the
    gradient scale; bf16 dh: within one bf16 ulp (+1e-6 absolute) of the exact value; dweight
    (f32 output, f32 sums): 1e-4 relative. Every element is written and reruns are bitwise equal."""
    h = normal(30 + rows % 7, (rows, dim), dtype)
    w = normal(31, (dim,), "f32", loc=1.0, scale=0.1)
    dy = normal(32, (rows, dim), dtype)
    dd = normal(33, (rows, dim), dtype) if direct else None
    ht, wt, gt = to_dev(h, dtype, dev), to_dev(w, "f32", dev), to_dev(dy, dtype, dev)
    dt = to_dev(dd, dtype, dev) if direct else None
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dh, dw = _bwd_abi(ht, wt, gt, dt, tdt)
    dh2, dw2 = _bwd_abi(ht, wt, gt, dt, tdt)
    assert not torch.isnan(dh).any() and not torch.isnan(dw).any()
    assert torch.equal(dh, dh2) and torch.equal(dw, dw2)
    ref_dh, ref_dw = orms.rmsnorm_bwd(h, w, dy)
    if direct:
        ref_dh = ref_dh + dd
    got = to_np(dh).astype(np.float64)
    if dtype == "bf16":
        assert np.all(np.abs(got - ref_dh) <= bf16_ulp(ref_dh.astype(np.float32)) + 1e-6)
    else:
        assert max_abs(got, ref_dh) <= 1e-4 * max(1.0, np.abs(ref_dh).max())
    assert max_abs(to_np(dw), ref_dw) <= 1e-4 * max(1.0, np.abs(ref_dw).max())


def test_bwd_kernel_f32_dh_from_bf16_and_zero_rows(dev):
    """dh in f32 from bf16 inputs (the mixed-residual case) and rows == 0 (dweight is zero)."""
    h, dy = normal(40, (64, 256), "bf16"), normal(41, (64, 256), "bf16")
    w = normal(42, (256,), "bf16", loc=1.0, scale=0.1)
    dh, dw = _bwd_abi(to_dev(h, "bf16", dev), to_dev(w, "bf16", dev), to_dev(dy, "bf16", dev), None, torch.float32)
    ref_dh, ref_dw = orms.rmsnorm_bwd(h, w, dy)
    assert dh.dtype == torch.float32 and max_abs(to_np(dh), ref_dh) <= 1e-4 * np.abs(ref_dh).max()
    assert np.all(np.abs(to_np(dw) - ref_dw) <= bf16_ulp(ref_dw.astype(np.float32)) + 1e-6)
    empty = torch.empty((0, 256), dtype=torch.bfloat16, device=dev)
    _, dw0 = _bwd_abi(empty, to_dev(w, "bf16", dev), empty, None, torch.bfloat16)
    assert torch.count_nonzero(dw0) == 0


def test_bf16_autograd_uses_the_kernel(dev):
    """Through rmsnorm(...).backward() in bf16 with an f32 weight (the GPT's layout): dx, dr and
    dweight within the bf16 bar of the f64 backward of the rounded h."""
    x, r = normal(50, (512, 768), "bf16"), normal(51, (512, 768), "bf16")
    w = normal(52, (768,), "f32", loc=1.0, scale=0.1)
    cot_y, cot_h = normal(53, (512, 768), "bf16"), normal(54, (512, 768), "bf16")
    xt, rt = to_dev(x, "bf16", dev).requires_grad_(), to_dev(r, "bf16", dev).requires_grad_()
    wt = to_dev(w, "f32", dev).requires_grad_()
    h, y = rmsnorm(xt, wt, residual=rt)
    torch.autograd.backward([y, h], [to_dev(cot_y, "bf16", dev), to_dev(cot_h, "bf16", dev)])
    hh = round_bf16(x + r)
    ref_dh, ref_dw = orms.rmsnorm_bwd(hh, w, cot_y)
    ref_dh = ref_dh + cot_h
    for g in (xt.grad, rt.grad):
        assert max_abs(to_np(g), ref_dh) <= 2e-2
    assert max_abs(to_np(wt.grad), ref_dw) <= 1e-3 * np.abs(ref_dw).max()


@pytest.mark.parametrize("nbytes", [16, 2048, 2048 * 1000 + 48, 4096 * 1024 * 2])
def test_stream_copy2_is_exact(dev, nbytes):
    """ferrite_hip_stream_copy2 (the streaming ceiling bench.py measures beside add+RMSNorm) copies
    both buffers bitwise, partial 2 KB units included, and writes nothing past them."""
    from ferrite import _hip

    n = nbytes // 4
    g = torch.Generator(device=dev).manual_seed(5)
    a = torch.randint(-2**31, 2**31 - 1, (n,), generator=g, device=dev, dtype=torch.int32)
    b = torch.randint(-2**31, 2**31 - 1, (n,), generator=g, device=dev, dtype=torch.int32)
    ao = torch.full((n + 64,), 7, device=dev, dtype=torch.int32)
    bo = torch.full((n + 64,), 7, device=dev, dtype=torch.int32)
    rc = _hip.lib().ferrite_hip_stream_copy2(a.data_ptr(), b.data_ptr(), ao.data_ptr(), bo.data_ptr(), nbytes,
                                             _hip.stream_of(a))
    _hip.check(rc, "stream_copy2")
    torch.cuda.synchronize()
    assert torch.equal(ao[:n], a) and torch.equal(bo[:n], b)
    assert bool((ao[n:] == 7).all()) and bool((bo[n:] == 7).all())


@pytest.mark.parametrize("blocks", [0, 1, 7, 1024])
@pytest.mark.parametrize("nbytes", [16, 4096, 4096 * 37 + 48, 3 << 20])
def test_stream_read_and_fill_are_exact(dev, nbytes, blocks):
    """The one-direction streams bench.py measures as HBM ceilings: ferrite_hip_stream_read leaves
    one word per workgroup whose XOR over the workgroups is the XOR of every word of the buffer
    (every byte read, partial 4 KB units included), and ferrite_hip_stream_fill writes `value` into
    every word and nothing past them."""
    from ferrite import _hip

    lib = _hip.lib()
    n = nbytes // 4
    g = torch.Generator(device=dev).manual_seed(11)
    a = torch.randint(-2**31, 2**31 - 1, (n,), generator=g, device=dev, dtype=torch.int32)
    units = nbytes // 4096
    used = max(1, min(blocks or 512, -(-units // 4)))  # the launch's workgroup count
    sink = torch.zeros(1024, device=dev, dtype=torch.int32)
    _hip.check(lib.ferrite_hip_stream_read(a.data_ptr(), nbytes, sink.data_ptr(), blocks, _hip.stream_of(a)),
               "stream_read")
    torch.cuda.synchronize()
    words = a.cpu().numpy().view(np.uint32)
    folded = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)[:used])
    assert int(folded) == int(np.bitwise_xor.reduce(words))
    out = torch.full((n + 64,), 7, device=dev, dtype=torch.int32)
    _hip.check(lib.ferrite_hip_stream_fill(out.data_ptr(), nbytes, 0x3F803F80, blocks, _hip.stream_of(a)), "fill")
    torch.cuda.synchronize()
    o = out.cpu().numpy().view(np.uint32)
    assert np.all(o[:n] == 0x3F803F80) and np.all(o[n:] == 7)

