"""Pins of the CPU oracle (CPU only). Every oracle function is checked against
something that does not share its code: a library routine, a closed form, an
invariant, brute force on tiny inputs, or an independent derivation."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import matmul as omm
from oracle import rmsnorm as orms
from oracle.bf16 import bits, from_bits, round_bf16
from tests._util import normal, rel_fro, uniform

# ---------------------------------------------------------------- bf16 rounding


def test_round_bf16_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32),
        (rng.standard_normal(10_000) * 1e30).astype(np.float32),
        (rng.standard_normal(10_000) * 1e-38).astype(np.float32),  # subnormals
        rng.integers(0, 2**32, 50_000, dtype=np.uint64).astype(np.uint32).view(np.float32),  # every bit pattern class
    ])
    x = x[~np.isnan(x)]
    ours = round_bf16(x)
    lib = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours.view(np.uint32), lib.view(np.uint32))


def test_round_bf16_ties_to_even_and_specials():
    one = np.float32(1.0)
    ulp = np.float32(2.0**-7)  # bf16 spacing at 1
    # exactly half an ulp above 1 -> ties to even (1); 1.5 ulp -> rounds up to 2 ulp (even)
    assert round_bf16(np.array([one + ulp / 2]))[0] == one
    assert round_bf16(np.array([one + 3 * ulp / 2]))[0] == one + 2 * ulp
    assert round_bf16(np.array([np.inf]))[0] == np.inf
    assert round_bf16(np.array([-np.inf]))[0] == -np.inf
    assert np.isnan(round_bf16(np.array([np.nan]))[0])
    # largest finite f32 rounds to inf in bf16 (as the library cast does)
    big = np.array([np.finfo(np.float32).max], np.float32)
    assert round_bf16(big)[0] == torch.from_numpy(big).to(torch.bfloat16).float().item()
    b = bits(round_bf16(np.array([1.0, -2.0], np.float32)))
    assert b.tolist() == [0x3F80, 0xC000]
    np.testing.assert_array_equal(from_bits(b), np.array([1.0, -2.0], np.float32))


# ---------------------------------------------------------------- rmsnorm


def test_rmsnorm_h_is_bf16_of_exact_sum():
    x = normal(0, (64, 256), "bf16")
    r = normal(1, (64, 256), "bf16")
    w = np.ones(256, np.float32)
    h, _ = orms.add_rmsnorm(x, w, r, out_bf16=True)
    # bf16 + bf16 is exact in f64; RNE of that must equal the oracle's h.
    exact = x.astype(np.float64) + r.astype(np.float64)
    lib = torch.from_numpy(exact).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(h, lib)


def test_rmsnorm_unit_rms_at_zero_eps():
    x = normal(2, (16, 384))
    y = orms.add_rmsnorm(x, np.ones(384, np.float32), eps=0.0, acc=np.float64)
    np.testing.assert_allclose(np.mean(y.astype(np.float64) ** 2, axis=-1), 1.0, rtol=1e-6)


def test_rmsnorm_constant_rows_closed_form():
    c = np.array([[3.0] * 8, [-0.5] * 8], np.float32)
    w = np.arange(1, 9, dtype=np.float32)
    eps = 1e-6
    y = orms.add_rmsnorm(c, w, eps=eps, acc=np.float64)
    expect = np.sign(c) * np.abs(c) / np.sqrt(c**2 + eps) * w
    np.testing.assert_allclose(y, expect, rtol=1e-6)


def test_rmsnorm_scale_invariance_and_f32_vs_f64():
    x = normal(3, (32, 1024))
    w = normal(4, (1024,), loc=1.0, scale=0.1)
    y1 = orms.add_rmsnorm(x, w, eps=0.0)
    y2 = orms.add_rmsnorm(np.float32(7.5) * x, w, eps=0.0)
    np.testing.assert_allclose(y1, y2, rtol=2e-6, atol=2e-6)
    y64 = orms.add_rmsnorm(x, w, eps=1e-6, acc=np.float64)
    np.testing.assert_allclose(orms.add_rmsnorm(x, w, eps=1e-6), y64, rtol=2e-6, atol=2e-6)


def test_rmsnorm_bwd_matches_autograd():
    h = normal(5, (8, 64)).astype(np.float64)
    w = normal(6, (64,), loc=1.0, scale=0.1).astype(np.float64)
    dy = normal(7, (8, 64)).astype(np.float64)
    ht = torch.tensor(h, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    y = ht * torch.rsqrt(torch.mean(ht * ht, -1, keepdim=True) + 1e-6) * wt
    (y * torch.tensor(dy)).sum().backward()
    dh, dw = orms.rmsnorm_bwd(h, w, dy, 1e-6)
    np.testing.assert_allclose(dh, ht.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, wt.grad.numpy(), rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------- attention


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("sq,sk", [(8, 8), (5, 7)])
def test_attention_forward_matches_brute_force(causal, sq, sk):
    if causal and sq != sk:
        sk = sq
    q, k, v = normal(10, (1, 2, sq, 8)), normal(11, (1, 2, sk, 8)), normal(12, (1, 2, sk, 8))
    o, lse = oatt.forward(q, k, v, causal=causal)
    ob, lb = oatt.brute_force(q, k, v, causal=causal)
    np.testing.assert_allclose(o, ob, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, lb, rtol=1e-12, atol=1e-12)


def test_attention_closed_forms():
    b, h, s, d = 1, 2, 16, 8
    q, k, v = normal(13, (b, h, s, d)), normal(14, (b, h, s, d)), normal(15, (b, h, s, d))
    o, _ = oatt.forward(q, k, v, causal=True)
    np.testing.assert_array_equal(o[:, :, 0], v[:, :, 0].astype(np.float64))  # row 0 sees key 0 only
    vc = np.broadcast_to(np.arange(d, dtype=np.float32), (b, h, s, d))
    oc, _ = oatt.forward(q, k, vc, causal=True)
    np.testing.assert_allclose(oc, vc, rtol=1e-12)  # convex combination of equal rows
    z = np.zeros_like(q)
    oz, lz = oatt.forward(z, k, v, causal=True)  # uniform weights over the i+1 visible keys
    cm = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, s + 1)[None, None, :, None]
    np.testing.assert_allclose(oz, cm, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lz, np.broadcast_to(np.log(np.arange(1, s + 1)), (b, h, s)), rtol=1e-12)


def test_attention_invariances():
    q, k, v = normal(16, (1, 1, 64, 16)), normal(17, (1, 1, 64, 16)), normal(18, (1, 1, 64, 16))
    full, _ = oatt.forward(q, k, v, causal=True)
    short, _ = oatt.forward(q[:, :, :32], k[:, :, :32], v[:, :, :32], causal=True)
    np.testing.assert_allclose(full[:, :, :32], short, rtol=1e-12, atol=1e-12)
    perm = np.random.default_rng(0).permutation(64)
    a, _ = oatt.forward(q, k, v, causal=False)
    b_, _ = oatt.forward(q, k[:, :, perm], v[:, :, perm], causal=False)
    np.testing.assert_allclose(a, b_, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_backward_matches_autograd(causal):
    q, k, v, do = (normal(20 + i, (1, 2, 24, 16)) for i in range(4))
    dq, dk, dv = oatt.backward(q, k, v, do, causal=causal)
    qt, kt, vt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v))
    s = qt @ kt.transpose(-1, -2) / math.sqrt(16)
    if causal:
        s = s.masked_fill(~torch.ones(24, 24, dtype=torch.bool).tril(), float("-inf"))
    out = torch.softmax(s, -1) @ vt
    (out * torch.tensor(do, dtype=torch.float64)).sum().backward()
    for ours, ref in zip((dq, dk, dv), (qt.grad, kt.grad, vt.grad)):
        np.testing.assert_allclose(ours, ref.numpy(), rtol=1e-10, atol=1e-12)


def test_attention_backward_matches_finite_differences():
    q, k, v, do = (normal(30 + i, (1, 1, 6, 4)) for i in range(4))
    dq, dk, dv = oatt.backward(q, k, v, do, causal=True)

    def loss(qq, kk, vv):
        o, _ = oatt.forward(qq, kk, vv, causal=True)
        return float(np.sum(o * do.astype(np.float64)))

    eps = 1e-6
    for grad, which in ((dq, 0), (dk, 1), (dv, 2)):
        args = [q.astype(np.float64), k.astype(np.float64), v.astype(np.float64)]
        num = np.zeros_like(args[which])
        for idx in np.ndindex(*args[which].shape):
            plus = [a.copy() for a in args]
            minus = [a.copy() for a in args]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            num[idx] = (loss(*plus) - loss(*minus)) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("causal", [True, False])
def test_flash_restatement_matches_materialised(causal):
    q, k, v, do = (normal(40 + i, (1, 2, 256, 64)) for i in range(4))
    o, lse = oatt.flash_forward(q, k, v, causal=causal, bq=64, bk=128)
    o_ref, lse_ref = oatt.forward(q, k, v, causal=causal)
    np.testing.assert_allclose(o, o_ref, atol=2e-6, rtol=2e-6)
    np.testing.assert_allclose(lse, lse_ref, atol=2e-6, rtol=2e-6)
    dq, dk, dv = oatt.flash_backward(q, k, v, do, o, lse, causal=causal, bq=64, bk=128)
    for a, b in zip((dq, dk, dv), oatt.backward(q, k, v, do, causal=causal)):
        np.testing.assert_allclose(a, b, atol=2e-5, rtol=2e-5)
    # bf16 variant: same recipe with P / dS rounded; stays within the bf16 bar of the exact result
    qb, kb, vb, dob = (round_bf16(a) for a in (q, k, v, do))
    ob, lb = oatt.flash_forward(qb, kb, vb, causal=causal, bq=64, bk=128, bf16=True)
    oe, le = oatt.forward(qb, kb, vb, causal=causal)
    assert np.max(np.abs(ob - oe)) < 2e-2
    assert np.max(np.abs(lb - le)) < 1e-3


# ---------------------------------------------------------------- matmul


def test_matmul_reference_matches_numpy_and_identity():
    x, y = uniform(50, (33, 47)), uniform(51, (47, 29))
    np.testing.assert_allclose(omm.reference(x, y), (x.astype(np.float64) @ y.astype(np.float64)).astype(np.float32))
    eye = np.eye(47, dtype=np.float32)
    np.testing.assert_array_equal(omm.reference(x, eye), x)


def test_matmul_blocked_padded_is_exact_on_integers():
    rng = np.random.default_rng(52)
    x = rng.integers(-8, 9, (77, 130)).astype(np.float32)
    y = rng.integers(-8, 9, (130, 203)).astype(np.float32)
    exact = (x.astype(np.int64) @ y.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(omm.blocked_padded(x, y, bm=64, bn=128, bk=128), exact)
    np.testing.assert_array_equal(omm.reference(x, y), exact)


def test_matmul_blocked_padded_close_on_floats():
    x, y = uniform(53, (100, 300)), uniform(54, (300, 70))
    assert rel_fro(omm.blocked_padded(x, y, bm=64, bn=128, bk=128), omm.reference(x, y)) < 1e-6
