"""GPU tests of the GELU matmul epilogues (csrc/matmul.hip: ferrite_hip_matmul_gelu) and the
fused MLP built on them (ferrite.kernels.matmul.mlp_gelu), the model's gelu(y @ w1) @ w2
(reference: src/ferrite/model/gpt.py:141, jax.nn.gelu(approximate=True)).

Pins: the pre-activation the forward stores is bitwise the plain product of the same kernel
(ferrite_hip_matmul_ex, same accumulation); gelu and gelu' are checked against torch's f64
tanh GELU and its autograd derivative (not against the kernel's own formulas), to one bf16 ulp
of the exact value; the fused MLP's output and gradients match the unfused composition
(matmul, torch's GELU, matmul) to the bf16 bar. Shapes cover the 128-row tiles, the 256-row
tiles, the K split (epilogue in the reduction) and the elementwise fallback for shapes the
DMA kernel does not take.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ferrite import _hip
from ferrite.kernels.matmul import matmul, mlp_gelu
from tests._util import bf16_ulp, normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _gelu64(u):
    return F.gelu(torch.from_numpy(u.astype(np.float64)), approximate="tanh").numpy()


def _gelu_grad64(u):
    t = torch.from_numpy(u.astype(np.float64)).requires_grad_()
    (g,) = torch.autograd.grad(F.gelu(t, approximate="tanh").sum(), t)
    return g.numpy()


def _fwd_bar(exact, u):
    """One bf16 ulp of the exact value, plus f32 rounding: 1e-6 relative, and 2^-23 |u| for the
    cancellation in 1 + tanh(...) at very negative u (where f32, as in torch, gives 0)."""
    return bf16_ulp(exact) + 1e-6 * np.abs(exact) + 2.0**-23 * np.abs(u) + 1e-30


def _call(x, y, m, n, k, x_t, y_t, mode, aux, workspace=True):
    lib = _hip.lib()
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=x.device)
    ws_bytes = lib.ferrite_hip_matmul_workspace(m, n, k, _hip.BF16) if workspace else 0
    ws = torch.empty(((ws_bytes + 3) // 4,), device=x.device) if ws_bytes > 0 else None
    rc = lib.ferrite_hip_matmul_gelu(x.data_ptr(), y.data_ptr(), out.data_ptr(), aux.data_ptr(), m, n, k, int(x_t),
                                     int(y_t), mode, _hip.ptr(ws), max(ws_bytes, 0), _hip.stream_of(x))
    _hip.check(rc, "matmul_gelu")
    return out


def _plain(x, y, m, n, k, x_t, y_t, workspace=True):
    lib = _hip.lib()
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=x.device)
    ws_bytes = lib.ferrite_hip_matmul_workspace(m, n, k, _hip.BF16) if workspace else 0
    ws = torch.empty(((ws_bytes + 3) // 4,), device=x.device) if ws_bytes > 0 else None
    rc = lib.ferrite_hip_matmul_ex(x.data_ptr(), y.data_ptr(), out.data_ptr(), m, n, k, int(x_t), int(y_t), _hip.BF16,
                                   _hip.BF16, _hip.ptr(ws), max(ws_bytes, 0), _hip.stream_of(x))
    _hip.check(rc, "matmul_ex")
    return out


SHAPES = [
    (8192, 3072, 768),   # 128-row tiles (the GPT's up-projection)
    (4096, 4096, 256),   # 256-row tiles
    (768, 768, 4096),    # few tiles: K split, the epilogue runs in the reduction
    (300, 264, 128),     # ragged rows and columns on the DMA kernel
    (100, 72, 136),      # K % 64 != 0: plain product, then the elementwise pass
]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("x_t,y_t", [(False, False), (False, True), (True, False)])
def test_gelu_forward_epilogue(dev, m, n, k, x_t, y_t):
    a = normal(60 + m % 7, (m, k), "bf16")
    b = normal(61 + n % 5, (k, n), "bf16", scale=0.05)
    xs = to_dev(a.T.copy() if x_t else a, "bf16", dev)
    ys = to_dev(b.T.copy() if y_t else b, "bf16", dev)
    u = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=dev)
    if (x_t or y_t) and not (k % 64 == 0 and n % 8 == 0 and (not x_t or m % 8 == 0)):
        # transposed operands outside the DMA kernel's rule are an error, as in ferrite_hip_matmul_ex
        with pytest.raises(RuntimeError, match="transposed"):
            _call(xs, ys, m, n, k, x_t, y_t, _hip.GELU, u)
        return
    out = _call(xs, ys, m, n, k, x_t, y_t, _hip.GELU, u)
    want_u = _plain(xs, ys, m, n, k, x_t, y_t)
    torch.cuda.synchronize()
    assert torch.equal(u, want_u)  # same kernel, same accumulation: the pre-activation is the product
    un = to_np(u).astype(np.float64)
    exact = _gelu64(un)
    got = to_np(out).astype(np.float64)
    assert np.all(np.abs(got - exact) <= _fwd_bar(exact, un))


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gelu_grad_epilogue(dev, m, n, k):
    """out = bf16(g @ w^T) * gelu'(u): w read transposed in place as the backward does (given
    as [k, n] where the DMA kernel does not take the shape)."""
    g = normal(70 + m % 3, (m, k), "bf16")
    w = normal(71, (n, k), "bf16", scale=0.05)
    u = normal(72, (m, n), "bf16", scale=2.0)
    y_t = k % 64 == 0
    gs, ws_, ut = to_dev(g, "bf16", dev), to_dev(w if y_t else w.T.copy(), "bf16", dev), to_dev(u, "bf16", dev)
    u_before = ut.clone()
    out = _call(gs, ws_, m, n, k, False, y_t, _hip.GELU_GRAD, ut)
    prod = _plain(gs, ws_, m, n, k, False, y_t)
    torch.cuda.synchronize()
    assert torch.equal(ut, u_before)  # aux is an input in this mode
    p64, u64 = to_np(prod).astype(np.float64), to_np(ut).astype(np.float64)
    exact = p64 * _gelu_grad64(u64)
    got = to_np(out).astype(np.float64)
    assert np.all(np.abs(got - exact) <= bf16_ulp(exact) + 1e-6 * np.abs(exact) + 4e-7 * np.abs(p64) * (1 + u64**2))


def test_split_and_unsplit_agree(dev):
    """Without a workspace the few-tile shape does not split; both results hold the same bar."""
    m, n, k = 768, 768, 4096
    a, b = normal(80, (m, k), "bf16"), normal(81, (k, n), "bf16", scale=0.03)
    xs, ys = to_dev(a, "bf16", dev), to_dev(b, "bf16", dev)
    u1 = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    u2 = torch.empty_like(u1)
    o1 = _call(xs, ys, m, n, k, False, False, _hip.GELU, u1)
    o2 = _call(xs, ys, m, n, k, False, False, _hip.GELU, u2, workspace=False)
    torch.cuda.synchronize()
    for u, o in ((u1, o1), (u2, o2)):
        un = to_np(u).astype(np.float64)
        exact = _gelu64(un)
        assert np.all(np.abs(to_np(o).astype(np.float64) - exact) <= _fwd_bar(exact, un))
    # summation order only: one bf16 ulp plus twice the f32 accumulation bound
    a1, a2 = to_np(u1).astype(np.float64), to_np(u2).astype(np.float64)
    absb = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    assert np.all(np.abs(a1 - a2) <= bf16_ulp(np.maximum(np.abs(a1), np.abs(a2))) + 2.0**-19 * absb)


def test_argument_errors(dev):
    lib = _hip.lib()
    x = torch.zeros(64, 64, device=dev, dtype=torch.bfloat16)
    o = torch.empty_like(x)
    st = _hip.stream_of(x)
    assert lib.ferrite_hip_matmul_gelu(x.data_ptr(), x.data_ptr(), o.data_ptr(), o.data_ptr(), 64, 64, 64, 0, 0,
                                       _hip.GELU, None, 0, st) == 1
    assert "differ" in _hip.last_error()
    assert lib.ferrite_hip_matmul_gelu(x.data_ptr(), x.data_ptr(), o.data_ptr(), x.data_ptr(), 64, 64, 64, 0, 0, 3,
                                       None, 0, st) == 1
    assert "mode" in _hip.last_error()


@pytest.mark.parametrize("t,d,f", [(2048, 768, 3072), (384, 256, 1024), (200, 64, 136)])
def test_mlp_matches_unfused(dev, t, d, f):
    """mlp_gelu against matmul -> torch's tanh GELU -> matmul on the same bf16 values: output and
    the three gradients within the bf16 bar (2 ulp of the larger magnitude, relative Frobenius 1e-2)."""
    x = normal(90, (t, d), "bf16")
    w1 = normal(91, (d, f), "bf16", scale=d ** -0.5)
    w2 = normal(92, (f, d), "bf16", scale=f ** -0.5)
    g = normal(93, (t, d), "bf16")
    outs = []
    for fused in (True, False):
        xt, w1t, w2t = (to_dev(a, "bf16", dev).requires_grad_() for a in (x, w1, w2))
        if fused:
            y = mlp_gelu(xt, w1t, w2t)
        else:
            y = matmul(F.gelu(matmul(xt, w1t), approximate="tanh"), w2t)
        y.backward(to_dev(g, "bf16", dev))
        outs.append([to_np(v).astype(np.float64) for v in (y, xt.grad, w1t.grad, w2t.grad)])
    for name, a, b in zip(("y", "dx", "dw1", "dw2"), *outs):
        scale = np.abs(b).max()
        assert np.abs(a - b).max() <= 2 * 2.0**-8 * scale, name
        assert np.linalg.norm(a - b) <= 1e-2 * np.linalg.norm(b), name


def test_mlp_rejects_non_bf16(dev):
    x = torch.zeros(4, 8, device=dev)
    with pytest.raises(ValueError):
        mlp_gelu(x, torch.zeros(8, 16, device=dev), torch.zeros(16, 8, device=dev))
