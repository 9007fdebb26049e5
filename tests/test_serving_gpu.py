"""GPU tests of the decode-attention kernel (csrc/decode.hip) and the serving engine
(reference: src/ferrite/serving/engine.py, tests/test_serving.py:11-32).

Pins for the kernel: the reference's own math (engine.py:89-104: write the new
rows, f32 scores over keys <= pos masked with -1e30, softmax, P.V), restated in
torch on the same inputs, at positions on and across the 256-key chunk edges;
the caches hold the new rows at pos and nothing else changed; out-of-range
positions write nothing and give NaN; reruns are bitwise equal. For the engine:
greedy tokens equal re-running the full model per step (the reference's own
test), decode logits equal the full forward's, and graph replay equals eager.
"""

import math

import numpy as np
import pytest
import torch

from ferrite.kernels.decode_attention import decode_attention, decode_attention_reference
from ferrite.model.gpt import GPTConfig, forward, init_params
from ferrite.serving.engine import Engine, ServeConfig, decode_step, prefill, reference_greedy
from tests._util import bf16_ulp

pytestmark = pytest.mark.gpu


def _case(dev, b, h, L, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(dev, dtype)
    return mk(b, h, d), mk(b, h, d), mk(b, h, d), mk(b, h, L, d), mk(b, h, L, d)


@pytest.mark.parametrize("b,h,L,d,dtype,pos", [
    (2, 3, 1000, 64, torch.bfloat16, [0, 999]),
    (2, 3, 1000, 64, torch.bfloat16, [255, 256]),
    (3, 2, 600, 128, torch.bfloat16, [511, 1, 300]),
    (1, 2, 256, 128, torch.float32, [100]),       # one chunk: direct output
    (2, 1, 300, 256, torch.bfloat16, [257, 299]),
    (4, 12, 2048, 64, torch.float32, [2047, 1024, 3, 1500]),
    # 128 heads: 1024-key chunks (the grid within 512 workgroups)
    (4, 32, 4096, 128, torch.bfloat16, [4095, 1023, 1024, 2500]),
    (2, 64, 4096, 64, torch.float32, [0, 4095]),
    # 128 heads over 16384 keys: four 4096-key chunks; positions at chunk and
    # row-step edges (a step of loads covers 32 rows at D = 64)
    (2, 64, 16384, 64, torch.bfloat16, [16383, 4096]),
    (2, 64, 16384, 64, torch.bfloat16, [4095, 8223]),
    # 640 heads: one 1024-key chunk holds all 1000 keys (direct output)
    (4, 160, 1000, 64, torch.float32, [999, 0, 500, 31]),
])
def test_decode_attention_matches_reference(dev, b, h, L, d, dtype, pos):
    q, kn, vn, kc, vc = _case(dev, b, h, L, d, dtype, sum(pos) + L)
    p = torch.tensor(pos, dtype=torch.int32, device=dev)
    kc0, vc0 = kc.clone(), vc.clone()
    kr, vr = kc.clone(), vc.clone()
    ref = decode_attention_reference(q, kn, vn, kr, vr, p)
    out = decode_attention(q, kn, vn, kc, vc, p)
    torch.cuda.synchronize()
    assert torch.equal(kc, kr) and torch.equal(vc, vr)  # the new rows at pos, nothing else
    for i, pi in enumerate(pos):
        kc0[i, :, pi] = kn[i]
        vc0[i, :, pi] = vn[i]
    assert torch.equal(kc, kc0) and torch.equal(vc, vc0)
    # the reference output, in f64 for the tolerance: softmax weights in f32 on both sides
    ref64 = torch.stack([
        (torch.softmax(torch.einsum("hd,hkd->hk", q[i].double(), kr[i, :, : pi + 1].double()) / math.sqrt(d), -1)[..., None]
         * vr[i, :, : pi + 1].double()).sum(1) for i, pi in enumerate(pos)])
    got = out.double()
    if dtype == torch.float32:
        assert float((got - ref64).abs().max()) <= 1e-5
    else:
        r = ref64.cpu().numpy()
        assert np.all(np.abs(got.cpu().numpy() - r) <= bf16_ulp(r.astype(np.float32)) + 1e-5)
        assert float((out.float() - ref.float()).abs().max()) <= 2e-2
    again = decode_attention(q, kn, vn, kc.clone(), vc.clone(), p)
    assert torch.equal(out, again)


def test_decode_attention_out_of_range_position(dev):
    q, kn, vn, kc, vc = _case(dev, 2, 2, 512, 64, torch.bfloat16, 3)
    kc0, vc0 = kc.clone(), vc.clone()
    out = decode_attention(q, kn, vn, kc, vc, torch.tensor([-1, 512], dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
    assert torch.equal(kc, kc0) and torch.equal(vc, vc0)


CFG = GPTConfig(vocab_size=256, seq_len=256, d_model=256, n_head=2, n_layer=2, d_ff=512, dtype=torch.float32)
XLA = dict(attention="xla", norm="xla", linear="xla", loss="xla")


def test_engine_matches_reference_greedy(dev):
    """tests/test_serving.py:11-21 on the HIP kernels, f32: prefill and decode replayed from graphs."""
    params = init_params(0, CFG, device=dev)
    eng = Engine(params, CFG, ServeConfig(batch=2, max_len=256, buckets=(128,)))
    assert eng.n_compiles == 2 and eng._decode.graph is not None
    prompts = [[1, 2, 3, 4, 5, 6, 7, 8, 9, 10], [42, 7, 99]]
    gen, stats = eng.generate(prompts, max_new_tokens=6)
    assert gen.shape == (2, 6) and stats["ttft_ms"] > 0
    for i, p in enumerate(prompts):
        np.testing.assert_array_equal(gen[i], reference_greedy(params, CFG.replace(**XLA), p, 6))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_logits_match_full_forward(dev, dtype):
    """After a prefill, each decode step's logits equal the full model's logits at that position
    (f32: 1e-4; bf16: 3e-2, the bf16 activations of two different operation orders)."""
    cfg = CFG.replace(dtype=dtype, linear="pallas")
    params = init_params(1, cfg, device=dev)
    toks = [5, 17, 200, 3, 9, 77, 31]
    lengths = torch.tensor([4], dtype=torch.int32, device=dev)
    t = torch.tensor([toks[:4] + [0] * 60], device=dev)
    logits, kc, vc = prefill(params, t, lengths, cfg, 256)
    full = forward(params, torch.tensor([toks], device=dev), cfg)
    tol = 1e-4 if dtype == torch.float32 else 3e-2
    assert float((logits[0] - full[0, 3]).abs().max()) <= tol
    for step in range(4, len(toks)):
        lg = decode_step(params, torch.tensor([toks[step]], device=dev),
                         torch.tensor([step], dtype=torch.int32, device=dev), kc, vc, cfg)
        assert float((lg[0] - full[0, step]).abs().max()) <= tol, step


def test_graph_replay_matches_eager_engine(dev):
    """bf16, batch 3, two buckets: the graph-replayed engine and an eager one give the same tokens."""
    cfg = CFG.replace(dtype=torch.bfloat16, linear="pallas", n_head=4)
    params = init_params(2, cfg, device=dev)
    prompts = [[3, 1, 4, 1, 5], [9, 2, 6, 5, 3, 5, 8, 9, 7, 9] * 7, [2, 7]]
    a = Engine(params, cfg, ServeConfig(batch=3, max_len=256, buckets=(32, 128)))
    b = Engine(params, cfg, ServeConfig(batch=3, max_len=256, buckets=(32, 128), graphs=False))
    ga, _ = a.generate(prompts, 12)
    gb, _ = b.generate(prompts, 12)
    np.testing.assert_array_equal(ga, gb)
    ga2, _ = a.generate([p[:3] for p in prompts], 5)  # the small bucket, after the large one
    gb2, _ = b.generate([p[:3] for p in prompts], 5)
    np.testing.assert_array_equal(ga2, gb2)


def test_engines_built_after_dropped_ones(dev):
    """Engines are built, used and dropped in a loop, as the serving benchmark does: a dropped
    engine's graphs must be gone before the next engine captures (no graph may be destroyed
    during a capture), so each new engine still matches the eager one."""
    import gc
    import weakref

    cfg = CFG.replace(dtype=torch.bfloat16, n_head=4)
    params = init_params(3, cfg, device=dev)
    ref = Engine(params, cfg, ServeConfig(batch=2, max_len=128, buckets=(32,), graphs=False))
    want, _ = ref.generate([[1, 2, 3], [4, 5]], 6)
    for batch_kernels in ("pallas", "xla", "pallas"):
        eng = Engine(params, cfg, ServeConfig(batch=2, max_len=128, buckets=(32,), decode_kernels=batch_kernels))
        got, _ = eng.generate([[1, 2, 3], [4, 5]], 6)
        if batch_kernels == "pallas":
            np.testing.assert_array_equal(got, want)
        alive = weakref.ref(eng._decode)
        del eng
        assert alive() is None  # freed without waiting for the cycle collector
    gc.collect()


def test_engine_close_releases_graphs(dev):
    """Explicit lifetime: leaving a ``with Engine(...)`` block destroys every captured graph, and
    an engine built after that captures and serves as before."""
    cfg = CFG.replace(dtype=torch.bfloat16, n_head=4)
    params = init_params(3, cfg, device=dev)
    with Engine(params, cfg, ServeConfig(batch=2, max_len=128, buckets=(32,))) as eng:
        want, _ = eng.generate([[1, 2, 3], [4, 5]], 6)
        decode = eng._decode
        assert decode.graph is not None
    assert decode.graph is None and not eng._prefill
    with Engine(params, cfg, ServeConfig(batch=2, max_len=128, buckets=(32,))) as eng2:
        got, _ = eng2.generate([[1, 2, 3], [4, 5]], 6)
    np.testing.assert_array_equal(got, want)
