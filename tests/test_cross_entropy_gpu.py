"""GPU tests of the softmax cross-entropy kernels (csrc/loss.hip) behind the GPT's
loss (reference: src/ferrite/model/gpt.py:147-152, f32 log_softmax + target NLL,
mean over tokens, and its autodiff backward).

Pins: float64 logsumexp and softmax computed with numpy on the same logits, the
one-hot term at the target, the dloss scaling, NaN for an out-of-range target
(what the reference's take_along_axis fill gives), and torch's own
F.cross_entropy through autograd.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ferrite.kernels.cross_entropy import cross_entropy, cross_entropy_grad, cross_entropy_rows
from tests._util import bf16_ulp

pytestmark = pytest.mark.gpu


def _case(n, v, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    x = (scale * rng.standard_normal((n, v))).astype(np.float32)
    t = rng.integers(0, v, size=n).astype(np.int64)
    return x, t


def _ref(x, t):
    x64 = x.astype(np.float64)
    m = x64.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(x64 - m).sum(axis=1, keepdims=True)))[:, 0]
    loss = lse - x64[np.arange(len(t)), t]
    return loss, lse, np.exp(x64 - lse[:, None])


@pytest.mark.parametrize("n,v", [(256, 32768), (37, 1001), (5, 4), (300, 256)])
def test_rows_and_grad_match_float64(dev, n, v):
    x, t = _case(n, v, n + v)
    xt, tt = torch.from_numpy(x).to(dev), torch.from_numpy(t).to(dev)
    loss, lse = cross_entropy_rows(xt, tt)
    ref_loss, ref_lse, p = _ref(x, t)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=0, atol=2e-5 * max(1.0, np.abs(ref_lse).max()))
    np.testing.assert_allclose(loss.cpu().numpy(), ref_loss, rtol=0, atol=2e-5 * max(1.0, np.abs(ref_lse).max()))
    dloss = torch.tensor(2.5, device=dev)
    g_ref = p.copy()
    g_ref[np.arange(n), t] -= 1.0
    g_ref *= 2.5 / n
    g32 = cross_entropy_grad(xt, tt, lse, dloss, 1.0 / n, torch.float32).cpu().numpy()
    np.testing.assert_allclose(g32, g_ref, rtol=0, atol=5e-5 * 2.5 / n)
    g16 = cross_entropy_grad(xt, tt, lse, dloss, 1.0 / n, torch.bfloat16).float().cpu().numpy()
    assert np.all(np.abs(g16 - g_ref) <= bf16_ulp(g_ref.astype(np.float32)) + 1e-8 * 2.5 / n)


def test_out_of_range_target_is_nan(dev):
    x, t = _case(4, 64, 1)
    t[2] = 64
    loss, _ = cross_entropy_rows(torch.from_numpy(x).to(dev), torch.from_numpy(t).to(dev))
    l = loss.cpu().numpy()
    assert np.isnan(l[2]) and np.isfinite(l[[0, 1, 3]]).all()


def test_autograd_matches_torch(dev):
    x, t = _case(512, 4096, 7)
    a = torch.from_numpy(x).to(dev).requires_grad_()
    b = torch.from_numpy(x).to(dev).requires_grad_()
    tt = torch.from_numpy(t).to(dev)
    la = cross_entropy(a, tt)
    lb = F.cross_entropy(b, tt)
    assert float(la.detach()) == pytest.approx(float(lb.detach()), rel=1e-5)
    (3.0 * la).backward()
    (3.0 * lb).backward()
    torch.testing.assert_close(a.grad, b.grad, rtol=1e-4, atol=1e-8)


def test_validation(dev):
    with pytest.raises(ValueError):
        cross_entropy_rows(torch.zeros(4, 8, device=dev, dtype=torch.bfloat16), torch.zeros(4, dtype=torch.long, device=dev))
    with pytest.raises(ValueError):
        cross_entropy_rows(torch.zeros(4, 8, device=dev), torch.zeros(5, dtype=torch.long, device=dev))
