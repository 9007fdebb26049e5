"""CPU tests of the GPT caller (ferrite.model): parameter tree and count, data
batches, the learning-rate schedule, closed forms of the first AdamW step, the
torch ("xla") route end to end on CPU, the checkpoint round trip, and that the
kernel ("pallas") route refuses CPU tensors.

Reference tests: tests/test_model.py:38-60 (param count formula, synthetic
batches, short run reduces loss). The kernel-route agreement tests
(test_model.py:13-35) need a GPU and live in test_model_gpu.py.
"""

import json
import math

import numpy as np
import pytest
import torch

from ferrite.model import data as data_lib
from ferrite.model.gpt import GPTConfig, forward, init_params, leaves, loss_fn, named_leaves, param_count
from ferrite.model.train import TrainConfig, adamw_init, adamw_update, load_params, lr_at, train

TINY = GPTConfig(vocab_size=256, seq_len=128, d_model=256, n_head=2, n_layer=2, d_ff=512, dtype=torch.float32)
XLA = dict(attention="xla", norm="xla", linear="xla", loss="xla")


def test_param_count_matches_formula():
    params = init_params(0, TINY)
    d, f, L, V, S = TINY.d_model, TINY.d_ff, TINY.n_layer, TINY.vocab_size, TINY.seq_len
    expected = V * d + S * d + d + L * (2 * d + 3 * d * d + d * d + d * f + f * d)
    assert param_count(params) == expected


def test_baseline_train_config_flops():
    """The 12-layer BASELINE train step: 84.95 M non-embedding parameters and 5.88 TFLOP per
    step of 8 x 1024 tokens (gpt.py:155-163, train.py:131-133)."""
    from ferrite.model.gpt import flops_per_token

    cfg = GPTConfig(vocab_size=32768, seq_len=1024, d_model=768, n_head=12, n_layer=12, d_ff=3072)
    d, f, L = cfg.d_model, cfg.d_ff, cfg.n_layer
    nonembed = L * (2 * d + 4 * d * d + 2 * d * f) + d
    assert nonembed == 84_953_856
    fpt = flops_per_token(cfg, nonembed)
    assert fpt["attention"] == 4 * 1024 * 768 * 12 * 0.5
    step = 3 * fpt["total"] * 8 * 1024
    assert abs(step / 1e12 - 5.876) < 1e-3


def test_init_params_statistics_and_layout():
    cfg = TINY.replace(n_layer=4)
    params = init_params(3, cfg)
    names = [n for n, _ in named_leaves(params)]
    assert names[:6] == ["layers/0/ln1", "layers/0/ln2", "layers/0/w1", "layers/0/w2", "layers/0/wo", "layers/0/wqkv"]
    assert names[-3:] == ["ln_f", "pos_emb", "tok_emb"]
    assert params["layers"][0]["wqkv"].shape == (256, 768) and params["layers"][0]["w2"].shape == (512, 256)
    assert abs(float(params["tok_emb"].std()) - 0.02) < 1e-3
    assert abs(float(params["layers"][1]["wo"].std()) - 0.02 / math.sqrt(8)) < 5e-4
    assert torch.equal(params["ln_f"], torch.ones(256))
    again = init_params(3, cfg)
    assert all(torch.equal(a, b) for a, b in zip(leaves(params), leaves(again)))
    assert init_params(0, cfg, param_dtype=torch.bfloat16)["tok_emb"].dtype == torch.bfloat16


def test_synthetic_data_batches():
    corpus = data_lib.synthetic(20_000, seed=1)
    x, y = data_lib.get_batch(np.random.default_rng(0), corpus, 4, 16)
    assert x.shape == (4, 16) and y.shape == (4, 16)
    assert x.dtype == np.int32
    np.testing.assert_array_equal(x[:, 1:], y[:, :-1])


def test_synthetic_corpus_is_the_markov_chain():
    """Determinism and structure: every symbol is < 64, and outside the ~5% noise positions it
    is one of the three table successors of the previous two symbols."""
    n, seed = 50_000, 4
    a = data_lib.synthetic(n, seed)
    np.testing.assert_array_equal(a, data_lib.synthetic(n, seed))
    assert a.dtype == np.uint8 and a.max() < 64
    rng = np.random.default_rng(seed)
    table = rng.integers(0, 64, size=(64, 64, 3))
    start = rng.integers(0, 64, size=2)
    choice = rng.integers(0, 3, size=n)
    noisy = rng.random(n) < 0.05
    np.testing.assert_array_equal(a[:2], start)
    i = np.arange(2, n)
    follows = table[a[i - 2], a[i - 1], choice[i]] == a[i]
    assert follows[~noisy[2:]].all()
    assert 0.9 < follows.mean() < 1.0


def test_load_falls_back_to_synthetic(tmp_path, monkeypatch):
    monkeypatch.chdir(tmp_path)
    with pytest.raises(FileNotFoundError):
        data_lib.load_tinyshakespeare(str(tmp_path))
    tr, va = data_lib.split(data_lib.load("tinyshakespeare"))
    assert len(tr) == 900_000 and len(va) == 100_000


def test_lr_schedule():
    cfg = TrainConfig(steps=120, lr=1e-3, warmup=20)
    assert lr_at(0, cfg) == pytest.approx(1e-3 / 20)
    assert lr_at(19, cfg) == pytest.approx(1e-3)
    assert lr_at(20, cfg) == pytest.approx(1e-3)  # cosine at progress 0
    assert lr_at(70, cfg) == pytest.approx(0.55e-3)  # halfway: 0.1 + 0.9 * 0.5
    assert lr_at(120, cfg) == pytest.approx(1e-4)
    assert lr_at(500, cfg) == pytest.approx(1e-4)


def test_first_adamw_step_closed_form():
    """On step 1 the bias-corrected moments are g and g^2, so the update is
    lr_1 * (g / (|g| + eps) + wd * p) for matrices and lr_1 * g / (|g| + eps) for vectors;
    clipping rescales g and cannot change that. gnorm is the pre-clip global norm."""
    torch.manual_seed(0)
    params = {"a": torch.randn(4, 3), "b": torch.randn(5), "layers": [{"c": torch.randn(2, 2)}]}
    grads = {"a": torch.randn(4, 3), "b": torch.randn(5) * 3, "layers": [{"c": torch.zeros(2, 2)}]}
    p0 = {k: v.clone() for k, v in params.items() if k != "layers"}
    c0 = params["layers"][0]["c"].clone()
    gsave = {k: v.clone() for k, v in grads.items() if k != "layers"}
    cfg = TrainConfig(lr=1e-2, warmup=4, steps=10, weight_decay=0.1, clip=0.5, optimizer="foreach")
    state = adamw_init(params)
    params, state, gnorm = adamw_update(params, grads, state, cfg)
    lr1 = lr_at(1, cfg)
    want_norm = math.sqrt(float((gsave["a"] ** 2).sum() + (gsave["b"] ** 2).sum()))
    assert float(gnorm) == pytest.approx(want_norm, rel=1e-6)
    ga, gb = gsave["a"], gsave["b"]
    torch.testing.assert_close(params["a"], p0["a"] - lr1 * (ga / (ga.abs() + 1e-8) + 0.1 * p0["a"]), atol=1e-6, rtol=0)
    torch.testing.assert_close(params["b"], p0["b"] - lr1 * gb / gb.abs(), atol=1e-6, rtol=0)
    # zero gradient: only the decay moves a matrix
    torch.testing.assert_close(params["layers"][0]["c"], c0 * (1 - lr1 * 0.1), atol=1e-7, rtol=0)
    assert state["step"] == 1


def test_bf16_params_keep_f32_moments():
    params = {"w": torch.randn(8, 8).to(torch.bfloat16)}
    state = adamw_init(params)
    assert state["m"]["w"].dtype == torch.float32
    before = params["w"].clone()
    adamw_update(params, {"w": torch.randn(8, 8).to(torch.bfloat16)}, state,
                 TrainConfig(lr=1e-2, warmup=1, optimizer="foreach"))
    assert params["w"].dtype == torch.bfloat16 and not torch.equal(params["w"], before)


def test_xla_route_forward_on_cpu():
    cfg = TINY.replace(**XLA, n_layer=1)
    params = init_params(0, cfg)
    tokens = torch.randint(0, 256, (2, 128), generator=torch.Generator().manual_seed(1))
    logits = forward(params, tokens, cfg)
    assert logits.shape == (2, 128, 256) and logits.dtype == torch.float32
    # causal: the first 64 positions do not see the last 64 tokens
    other = tokens.clone()
    other[:, 64:] = (other[:, 64:] + 7) % 256
    torch.testing.assert_close(forward(params, other, cfg)[:, :64], logits[:, :64], atol=1e-5, rtol=1e-5)
    # near-uniform predictions at init (targets other than the input token, which the tied head favours)
    loss = loss_fn(params, tokens, (tokens + 1) % 256, cfg)
    assert abs(float(loss) - math.log(256)) < 0.1
    with pytest.raises(ValueError):
        forward(params, torch.zeros((1, 129), dtype=torch.long), cfg)


def test_kernel_route_refuses_cpu_tensors():
    params = init_params(0, TINY.replace(n_layer=1))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        forward(params, torch.zeros((1, 128), dtype=torch.long), TINY.replace(n_layer=1))
    grads = {k: v for k, v in params.items()}
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        adamw_update(params, grads, adamw_init(params), TrainConfig())  # the fused optimiser is HIP-only
    with pytest.raises(ValueError):
        TrainConfig(optimizer="sgd")


def test_config_validates_routes():
    with pytest.raises(ValueError):
        TINY.replace(attention="triton")
    assert TINY.attention_blocks(384).block_q == 128
    assert TINY.attention_blocks(100) is None


def test_short_training_run_reduces_loss_on_cpu(tmp_path):
    cfg = TINY.replace(seq_len=64, d_model=64, n_head=1, n_layer=1, d_ff=128, **XLA)
    tcfg = TrainConfig(steps=12, batch=8, lr=3e-3, warmup=2, log_every=100, data="synthetic",
                       out=str(tmp_path / "r.json"), save_params=str(tmp_path / "p.npz"), optimizer="foreach")
    res = train(cfg, tcfg, verbose=False, device="cpu")
    assert res["loss_last"] < res["loss_first"]
    assert res["tokens_per_second"] > 0 and res["mfu"] is None
    saved = json.loads((tmp_path / "r.json").read_text())
    assert saved["model"]["dtype"] == "float32" and saved["model"]["params"] == param_count(init_params(0, cfg))
    back = load_params(str(tmp_path / "p.npz"), cfg)
    assert [n for n, _ in named_leaves(back)] == [n for n, _ in named_leaves(init_params(0, cfg))]
    assert not torch.equal(back["tok_emb"], init_params(0, cfg)["tok_emb"])  # trained


def test_cli_on_cpu(tmp_path):
    """The command line (train.py:201-227 in the reference) runs the torch routes on the CPU and picks
    the multi-tensor optimizer there by default."""
    from ferrite.model.train import main

    out = tmp_path / "cli.json"
    main(["--steps", "2", "--batch", "2", "--seq", "32", "--layers", "1", "--d-model", "32", "--heads", "1",
          "--d-ff", "64", "--data", "synthetic", "--dtype", "float32", "--attention", "xla", "--norm", "xla",
          "--linear", "xla", "--loss", "xla", "--out", str(out)])
    res = json.loads(out.read_text())
    assert res["train"]["optimizer"] == "foreach" and res["model"]["loss"] == "xla"
    assert np.isfinite(res["loss_last"])
