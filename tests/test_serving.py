"""CPU tests of the serving engine (reference: tests/test_serving.py:11-36): bucket
selection, and the engine's prefill + cached decode against re-running the full model
each step, on the torch route (graphs off, on the CPU)."""

import numpy as np
import pytest
import torch

from ferrite.model.gpt import GPTConfig, init_params
from ferrite.serving.engine import Engine, ServeConfig, bucket_for, reference_greedy

CFG = GPTConfig(vocab_size=256, seq_len=256, d_model=128, n_head=1, n_layer=2, d_ff=256, dtype=torch.float32)
XLA = dict(attention="xla", norm="xla", linear="xla", loss="xla")


def test_bucket_selection():
    assert bucket_for(1, (64, 128)) == 64 and bucket_for(64, (64, 128)) == 64 and bucket_for(65, (64, 128)) == 128
    with pytest.raises(ValueError):
        bucket_for(129, (64, 128))


def test_engine_matches_reference_greedy_on_cpu():
    cfg = CFG.replace(**XLA)
    params = init_params(0, cfg)
    eng = Engine(params, cfg, ServeConfig(batch=2, max_len=256, buckets=(128,), prefill_kernels="xla",
                                          decode_kernels="xla", graphs=False))
    assert eng.n_compiles == 2  # one prefill bucket + decode
    prompts = [[1, 2, 3, 4, 5, 6, 7, 8, 9, 10], [42, 7, 99]]
    gen, stats = eng.generate(prompts, max_new_tokens=6)
    assert gen.shape == (2, 6) and stats["ttft_ms"] > 0
    for i, p in enumerate(prompts):
        np.testing.assert_array_equal(gen[i], reference_greedy(params, cfg, p, 6))


def test_engine_validation():
    params = init_params(0, CFG.replace(**XLA))
    with pytest.raises(ValueError):
        Engine(params, CFG.replace(**XLA), ServeConfig(max_len=512, graphs=False))
    eng = Engine(params, CFG.replace(**XLA), ServeConfig(batch=1, max_len=64, buckets=(32,), prefill_kernels="xla",
                                                         decode_kernels="xla", graphs=False))
    with pytest.raises(ValueError):
        eng.generate([[1] * 30], max_new_tokens=40)
    with pytest.raises(ValueError):
        eng.prefill([[1], [2]])


def test_closed_engine_refuses_to_serve():
    """close() ends an engine's use: prefill, decode and generate raise instead of failing deep
    inside (a missing bucket) or quietly capturing a new graph."""
    cfg = CFG.replace(**XLA)
    params = init_params(0, cfg)
    with Engine(params, cfg, ServeConfig(batch=1, max_len=64, buckets=(32,), prefill_kernels="xla",
                                         decode_kernels="xla", graphs=False)) as eng:
        tok, pos, _, _ = eng.prefill([[1, 2, 3]])
    for call in (lambda: eng.prefill([[1, 2, 3]]), lambda: eng.decode(tok, pos), lambda: eng.generate([[1, 2]], 2)):
        with pytest.raises(RuntimeError, match="engine closed"):
            call()
    eng.close()  # closing again is harmless


def test_capture_window_holds_off_the_cycle_collector():
    """ferrite.graphs.capture_window: no cyclic collection inside a capture, the collector's
    previous state restored afterwards (also when the capture raises)."""
    import gc

    from ferrite.graphs import capture_window

    assert gc.isenabled()
    with capture_window():
        assert not gc.isenabled()
    assert gc.isenabled()
    try:
        with capture_window():
            raise RuntimeError("capture failed")
    except RuntimeError:
        pass
    assert gc.isenabled()
    gc.disable()
    try:
        with capture_window():
            assert not gc.isenabled()
        assert not gc.isenabled()
    finally:
        gc.enable()
