"""GPU tests of the fused AdamW kernel (csrc/optim.hip) behind
ferrite.model.train.adamw_update (reference: src/ferrite/model/train.py:59-74).

Pins: the closed form of the first step (bias-corrected moments are g and g^2,
so the step is lr * (g/(|g|+eps) + decay*p)); the global norm against torch's;
and several steps against the torch multi-tensor route of the same update,
which the CPU tests pin by the same closed forms. Tensor lists cover several
kernel-argument groups (more than 32 tensors), ragged sizes (numel % 8 != 0),
a misaligned tensor (the scalar path) and empty tensors.
"""

import math

import numpy as np
import pytest
import torch

from ferrite.kernels.adamw import fused_adamw_
from ferrite.model.train import TrainConfig, adamw_init, adamw_update, lr_at
from tests._util import bf16_ulp

pytestmark = pytest.mark.gpu

SHAPES = [(768, 2304), (768,), (3, 5), (7,), (0,), (1,), (64, 64), (1000,), (33, 17)] + [(40 + i,) for i in range(30)]


def _tree(dev, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    leaves = [(scale * torch.randn(s, generator=g)).to(dev, dtype) for s in SHAPES]
    # a contiguous tensor whose data pointer is not 16-byte aligned (element offset 1)
    base = (scale * torch.randn(1 + 501, generator=g)).to(dev, dtype)
    leaves.append(base[1:])
    return {"layers": [{"w": t} for t in leaves]}


def test_first_step_closed_form(dev):
    params = _tree(dev, torch.float32, 0)
    grads = _tree(dev, torch.float32, 1)
    p0 = [l["w"].clone() for l in params["layers"]]
    g0 = [l["w"].clone() for l in grads["layers"]]
    cfg = TrainConfig(lr=1e-2, warmup=4, steps=10, weight_decay=0.1, clip=0.5)
    state = adamw_init(params)
    params, state, gnorm = adamw_update(params, grads, state, cfg)
    want = math.sqrt(sum(float((g.double() ** 2).sum()) for g in g0))
    assert float(gnorm) == pytest.approx(want, rel=1e-5)
    lr1 = lr_at(1, cfg)
    scale = min(1.0, 0.5 / (want + 1e-6))
    for l, p, g in zip(params["layers"], p0, g0):
        decay = 0.1 if p.ndim >= 2 else 0.0
        gs = g * scale
        exp = p - lr1 * (gs / (gs.abs() + 1e-8) + decay * p)
        torch.testing.assert_close(l["w"], exp, atol=2e-6, rtol=0)
    assert state["step"] == 1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("clip", [1.0, 1e3, 0.0])
def test_matches_foreach_route_over_steps(dev, dtype, clip):
    """Five steps of the fused kernel against the torch multi-tensor route from the same state:
    f32 parameters within 1e-5 relative, bf16 parameters within one bf16 ulp, moments 1e-5
    relative (1e-6 of the tensor's largest moment absolute)."""
    pa, pb = _tree(dev, dtype, 3, 0.05), _tree(dev, dtype, 3, 0.05)
    sa, sb = adamw_init(pa), adamw_init(pb)
    fused = TrainConfig(lr=3e-3, warmup=2, steps=20, weight_decay=0.1, clip=clip)
    ref = TrainConfig(lr=3e-3, warmup=2, steps=20, weight_decay=0.1, clip=clip, optimizer="foreach")
    for k in range(5):
        grads = _tree(dev, dtype, 10 + k, 0.3)
        grads2 = {"layers": [{"w": l["w"].clone()} for l in grads["layers"]]}
        pa, sa, na = adamw_update(pa, grads, sa, fused)
        pb, sb, nb = adamw_update(pb, grads2, sb, ref)
        assert float(na) == pytest.approx(float(nb), rel=1e-5)
    for la, lb, ma, mb, va, vb in zip(pa["layers"], pb["layers"], sa["m"]["layers"], sb["m"]["layers"],
                                      sa["v"]["layers"], sb["v"]["layers"]):
        a, b = la["w"].double().cpu().numpy(), lb["w"].double().cpu().numpy()
        if dtype == torch.float32:
            assert np.all(np.abs(a - b) <= 1e-5 * np.maximum(np.abs(b), 1e-2))
        else:
            assert np.all(np.abs(a - b) <= bf16_ulp(b.astype(np.float32)) + 1e-9)
        # moments: the two routes round b1*m + (1-b1)*g in different orders; near-cancelling
        # elements are compared on the scale of the tensor
        for x, y in ((ma["w"], mb["w"]), (va["w"], vb["w"])):
            if y.numel():
                torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-6 * float(y.abs().max()))


def test_direct_call_validates(dev):
    p = [torch.zeros(8, device=dev)]
    with pytest.raises(ValueError):
        fused_adamw_(p, [torch.zeros(9, device=dev)], [torch.zeros(8, device=dev)], [torch.zeros(8, device=dev)], [True],
                     lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.0, max_grad_norm=1.0, step=1)
    with pytest.raises(ValueError):
        fused_adamw_(p, [torch.zeros(8, device=dev)], [torch.zeros(8, device=dev, dtype=torch.bfloat16)],
                     [torch.zeros(8, device=dev)], [True],
                     lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.0, max_grad_norm=1.0, step=1)
