"""GPU tests of the GPT caller: the kernel ("pallas") route against the torch
("xla") route, forward and gradients, and short training runs.

Reference tests: tests/test_model.py:13-35 and :55-60, with the same TINY
config (f32) and tolerances: logits atol/rtol 2e-4 (attention + norm kernels),
5e-4 (matmul kernel as well), gradients atol 2e-4 / rtol 2e-3. The bf16 case
adds the 2e-2 max-abs bar of the bf16 kernel outputs.
"""

import math

import numpy as np
import pytest
import torch

from ferrite.model.gpt import GPTConfig, forward, init_params, leaves, loss_fn, named_leaves
from ferrite.model.train import TrainConfig, adamw_init, build_train_step, train, value_and_grad

pytestmark = pytest.mark.gpu

TINY = GPTConfig(vocab_size=256, seq_len=128, d_model=256, n_head=2, n_layer=2, d_ff=512, dtype=torch.float32)
XLA = dict(attention="xla", norm="xla", linear="xla", loss="xla")


def _tokens(dev, b=2, s=128, vocab=256, seed=1):
    return torch.randint(0, vocab, (b, s), generator=torch.Generator().manual_seed(seed)).to(dev)


def test_pallas_and_xla_paths_agree(dev):
    params = init_params(0, TINY, device=dev)
    tokens = _tokens(dev)
    out_pallas = forward(params, tokens, TINY)
    out_xla = forward(params, tokens, TINY.replace(attention="xla", norm="xla"))
    assert out_pallas.shape == (2, 128, 256)
    np.testing.assert_allclose(out_pallas.cpu().numpy(), out_xla.cpu().numpy(), atol=2e-4, rtol=2e-4)


def test_pallas_linear_path_agrees(dev):
    params = init_params(0, TINY, device=dev)
    tokens = _tokens(dev)
    a = forward(params, tokens, TINY.replace(linear="pallas"))
    b = forward(params, tokens, TINY.replace(**XLA))
    np.testing.assert_allclose(a.cpu().numpy(), b.cpu().numpy(), atol=5e-4, rtol=5e-4)


@pytest.mark.parametrize("linear", ["xla", "pallas"])
def test_gradients_agree_between_paths(dev, linear):
    params = init_params(0, TINY, device=dev)
    x = _tokens(dev)
    y = torch.roll(x, -1, dims=1)
    _, g1 = value_and_grad(params, x, y, TINY.replace(linear=linear))
    _, g2 = value_and_grad(params, x, y, TINY.replace(**XLA))
    for (name, a), b in zip(named_leaves(g1), leaves(g2)):
        np.testing.assert_allclose(a.cpu().numpy(), b.cpu().numpy(), atol=2e-4, rtol=2e-3, err_msg=name)


def test_bf16_routes_agree(dev):
    """bf16 activations, f32 parameters: all three kernels against torch math. Logits within the
    2e-2 bf16 bar; gradients point the same way (cosine > 0.99 per tensor)."""
    cfg = TINY.replace(dtype=torch.bfloat16, linear="pallas", seq_len=256, n_head=4)
    params = init_params(2, cfg, device=dev)
    x = _tokens(dev, b=2, s=256, seed=5)
    y = torch.roll(x, -1, dims=1)
    la = forward(params, x, cfg)
    lb = forward(params, x, cfg.replace(**XLA))
    assert la.dtype == torch.float32
    assert float((la - lb).abs().max()) <= 2e-2
    loss_a, ga = value_and_grad(params, x, y, cfg)
    loss_b, gb = value_and_grad(params, x, y, cfg.replace(**XLA))
    assert abs(float(loss_a) - float(loss_b)) < 1e-3
    for (name, a), b in zip(named_leaves(ga), leaves(gb)):
        a, b = a.double().flatten(), b.double().flatten()
        cos = float(a @ b / (a.norm() * b.norm() + 1e-30))
        assert cos > 0.99, (name, cos)


def test_short_training_run_reduces_loss(tmp_path):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    cfg = TINY.replace(seq_len=128, d_model=128, n_head=1, n_layer=1, d_ff=256)
    tcfg = TrainConfig(steps=12, batch=8, lr=3e-3, warmup=2, log_every=100, data="synthetic",
                       out=str(tmp_path / "r.json"), save_params=str(tmp_path / "p.npz"))
    res = train(cfg, tcfg, verbose=False)
    assert res["loss_last"] < res["loss_first"]
    assert (tmp_path / "r.json").exists() and (tmp_path / "p.npz").exists()
    assert res["tokens_per_second"] > 0


def test_bf16_training_on_kernels_tracks_the_torch_route():
    """60 bf16 steps on the synthetic corpus with all three kernels, and the same run on torch
    math: both learn its 64-symbol alphabet (loss from log(256) to about log(64)) and their
    loss curves stay within 0.05 of each other."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    cfg = GPTConfig(vocab_size=256, seq_len=128, d_model=256, n_head=2, n_layer=2, d_ff=512, linear="pallas")
    tcfg = TrainConfig(steps=60, batch=16, lr=3e-3, warmup=5, log_every=1000, data="synthetic")
    res = train(cfg, tcfg, verbose=False)
    ref = train(cfg.replace(**XLA), tcfg, verbose=False)
    assert res["loss_first"] > 5.0
    assert res["loss_last"] < math.log(64) + 0.15, res["loss_curve"]
    assert np.max(np.abs(np.array(res["loss_curve"]) - np.array(ref["loss_curve"]))) < 0.05


def test_baseline_train_step_config(dev):
    """BASELINE config 5 at its size: 12 layers, d_model 768, 12 heads of 64, MLP 3072, vocab
    32768, seq 1024, batch 8, bf16 parameters (N(0, 0.02) with the scaled residual projections),
    tokens U[0, vocab). The kernel route (attention, norms, matmul, loss on the HIP kernels) and
    the torch route start from the same parameters and tokens (tests/test_model.py:13-37 at this
    config): their losses agree within 1e-3 and every gradient tensor points the same way
    (cosine > 0.99). Then one forward+backward+AdamW step on the kernels: finite loss near
    log(vocab), finite gradient norm, every parameter moved."""
    cfg = GPTConfig(vocab_size=32768, seq_len=1024, d_model=768, n_head=12, n_layer=12, d_ff=3072, linear="pallas")
    params = init_params(0, cfg, device=dev, param_dtype=torch.bfloat16)
    x = _tokens(dev, b=8, s=1024, vocab=32768, seed=9)
    y = torch.roll(x, -1, dims=1)
    loss_a, ga = value_and_grad(params, x, y, cfg)
    loss_b, gb = value_and_grad(params, x, y, cfg.replace(**XLA))
    assert abs(float(loss_a) - float(loss_b)) < 1e-3, (float(loss_a), float(loss_b))
    for (name, a), b in zip(named_leaves(ga), leaves(gb)):
        a, b = a.double().flatten(), b.double().flatten()
        cos = float(a @ b / (a.norm() * b.norm() + 1e-30))
        assert cos > 0.99, (name, cos)
    del ga, gb
    before = [t.clone() for t in leaves(params)]
    opt = adamw_init(params)
    step = build_train_step(cfg, TrainConfig(steps=10, warmup=1, lr=1e-2))  # bf16 gains of 1.0 need steps above 2^-8
    params, opt, loss, gnorm = step(params, opt, x, y)
    assert abs(float(loss) - math.log(32768)) < 0.5
    assert abs(float(loss) - float(loss_b)) < 1e-3
    assert math.isfinite(float(gnorm)) and float(gnorm) > 0
    for (name, t), b in zip(named_leaves(params), before):
        assert not torch.equal(t, b), name


@pytest.mark.parametrize("linear", ["pallas", "xla"])
def test_graphed_step_matches_eager(dev, linear):
    """The HIP-graph train step against the eager one, one step at a time from the same state:
    before every step the eager tree is set to the graphed run's parameters and moments, then both
    take the step on the same tokens (two eager warm-up calls, the capture, then replays with
    eager work and synchronisations in between). Each step's loss, gradient norm, parameters
    and moments must agree to 1e-6. A step moves parameters by ~lr = 3e-3 and the schedule's
    lr changes by ~1e-4 per step here, so stale per-step values or a corrupted replay would
    fail by orders of magnitude. (The runs are not compared as whole trajectories: the tied
    head's products run on the library GEMM, and Adam amplifies last-bit differences of
    near-cancelling moments over steps.)"""
    cfg = GPTConfig(vocab_size=256, seq_len=128, d_model=256, n_head=2, n_layer=2, d_ff=512, linear=linear)
    tcfg = TrainConfig(steps=10, warmup=2, lr=3e-3)
    pa, pb = init_params(4, cfg, device=dev), init_params(4, cfg, device=dev)
    sa, sb = adamw_init(pa), adamw_init(pb)
    eager = build_train_step(cfg, tcfg)
    graphed = build_train_step(cfg, tcfg, graph=True)
    g = torch.Generator().manual_seed(6)
    for i in range(6):
        with torch.no_grad():
            for a, b in zip(leaves(pa) + leaves(sa["m"]) + leaves(sa["v"]), leaves(pb) + leaves(sb["m"]) + leaves(sb["v"])):
                a.copy_(b)
        sa["step"] = sb["step"]
        x = torch.randint(0, 256, (4, 128), generator=g).to(dev)
        y = torch.randint(0, 256, (4, 128), generator=g).to(dev)
        pa, sa, la, na = eager(pa, sa, x, y)
        pb, sb, lb, nb = graphed(pb, sb, x, y)
        la, lb = float(la), float(lb)
        torch.cuda.synchronize()
        assert abs(la - lb) <= 1e-6 * abs(la), (i, la, lb)
        assert abs(float(na) - float(nb)) <= 1e-5 * float(na), (i, float(na), float(nb))
        for (name, a), b in zip(named_leaves({"p": pa, "m": sa["m"], "v": sa["v"]}),
                                leaves({"p": pb, "m": sb["m"], "v": sb["v"]})):
            d = float((a.detach().float() - b.detach().float()).abs().max())
            assert d <= 1e-6, (i, name, d)
    assert graphed.graph is not None and sb["step"] == 6
