"""The allocation-free RMSNorm backward (ferrite_hip_rmsnorm_bwd_noalloc) against the workspace
entry point it shares its kernels with (ferrite_hip_rmsnorm_bwd), through the C ABI.

Same kernels, same partial-row layout, same fixed summation order: dh and dweight must be
bitwise equal. The scratch array keeps the previous call's contents, so each case runs two
calls in a row, the second on a smaller input, and both are checked. A shape needing more
scratch than the array holds is refused with an error (and writes nothing)."""

import numpy as np
import pytest
import torch

from ferrite import _hip
from tests._util import normal, to_dev

pytestmark = pytest.mark.gpu


def _inputs(dev, rows, dim, xd, wd, direct, seed):
    h = to_dev(normal(seed, (rows, dim), xd), xd, dev)
    dy = to_dev(normal(seed + 1, (rows, dim), xd), xd, dev)
    w = to_dev(normal(seed + 2, (dim,), wd, scale=0.1, loc=1.0), wd, dev)
    dd = to_dev(normal(seed + 3, (rows, dim), xd), xd, dev) if direct else None
    return h, dy, w, dd


def _run(dev, h, dy, w, dd, rows, dim, xd, wd, od, noalloc):
    lib, st = _hip.lib(), _hip.stream_of(h)
    dh = torch.full((rows, dim), float("nan"), dtype=torch.float32 if od == "f32" else torch.bfloat16, device=dev)
    dw = torch.full((dim,), float("nan"), dtype=w.dtype, device=dev)
    args = (h.data_ptr(), w.data_ptr(), dy.data_ptr(), None if dd is None else dd.data_ptr(), dh.data_ptr(),
            dw.data_ptr())
    codes = (_hip.dtype_code(h.dtype), _hip.dtype_code(w.dtype), _hip.F32 if od == "f32" else _hip.BF16)
    if noalloc:
        rc = lib.ferrite_hip_rmsnorm_bwd_noalloc(*args, rows, dim, *codes, 1e-6, st)
    else:
        ws = torch.empty((lib.ferrite_hip_rmsnorm_bwd_workspace(rows, dim) + 3) // 4, dtype=torch.float32,
                         device=dev)
        rc = lib.ferrite_hip_rmsnorm_bwd(*args, ws.data_ptr(), rows, dim, *codes, 1e-6, st)
    _hip.check(rc, "rmsnorm_bwd" + ("_noalloc" if noalloc else ""))
    torch.cuda.synchronize()
    return dh, dw


# (rows, dim) of the first call, then of the second, smaller call
@pytest.mark.parametrize("first,second,xd,wd,od,direct", [
    ((8192, 768), (1000, 512), "bf16", "f32", "bf16", True),   # the GPT step's norms, fast path
    ((8192, 4096), (64, 1024), "bf16", "bf16", "bf16", False),  # the largest fast-path dim: 512 x 4096 floats = 8 MiB
    ((3000, 1000), (77, 136), "f32", "f32", "f32", False),     # f32, fast path
    ((700, 100), (33, 60), "bf16", "f32", "f32", True),        # dim % 8 != 0: general row + column passes
])
def test_noalloc_matches_workspace_entry(dev, first, second, xd, wd, od, direct):
    for i, (rows, dim) in enumerate((first, second)):
        h, dy, w, dd = _inputs(dev, rows, dim, xd, wd, direct, seed=200 + 10 * i)
        ref_dh, ref_dw = _run(dev, h, dy, w, dd, rows, dim, xd, wd, od, noalloc=False)
        got_dh, got_dw = _run(dev, h, dy, w, dd, rows, dim, xd, wd, od, noalloc=True)
        assert not torch.isnan(got_dh.float()).any() and not torch.isnan(got_dw.float()).any()
        assert torch.equal(got_dh, ref_dh), (i, rows, dim)
        assert torch.equal(got_dw, ref_dw), (i, rows, dim)


def test_noalloc_refuses_shapes_beyond_its_scratch(dev):
    """dim 8192 is past the one-pass kernel's 4096, so 4112 rows take the general path: 512 partial
    rows of 8192 floats plus one float per row, (512 * 8192 + 4112) * 4 = 16.8 MB > 8 MiB. Refused
    before any launch, outputs untouched."""
    rows, dim = 4112, 8192
    h, dy, w, _ = _inputs(dev, rows, dim, "bf16", "f32", False, seed=230)
    dh = torch.full((rows, dim), float("nan"), dtype=torch.bfloat16, device=dev)
    dw = torch.full((dim,), float("nan"), dtype=torch.float32, device=dev)
    rc = _hip.lib().ferrite_hip_rmsnorm_bwd_noalloc(h.data_ptr(), w.data_ptr(), dy.data_ptr(), None, dh.data_ptr(),
                                                    dw.data_ptr(), rows, dim, _hip.BF16, _hip.F32, _hip.BF16, 1e-6,
                                                    _hip.stream_of(h))
    assert rc == 1 and "scratch" in _hip.last_error()
    torch.cuda.synchronize()
    assert torch.isnan(dw).all() and torch.isnan(dh.float()).all()
    np.testing.assert_equal(_hip.RMSNORM_BWD_SCRATCH_BYTES, 8 << 20)


def test_noalloc_scratch_edge_on_the_general_path(dev):
    """The refusal edge of the general path (dim % 8 != 0): nparts = min(rows, 512) partial rows of
    dim floats plus one float per row. dim 4095 with 512 rows needs (512 * 4095 + 512) * 4 bytes,
    exactly the 8 MiB array: accepted and bitwise equal to the workspace entry. 513 rows need four
    bytes more: refused, outputs untouched."""
    dim = 4095
    rows = 512
    assert (rows * dim + rows) * 4 == _hip.RMSNORM_BWD_SCRATCH_BYTES
    h, dy, w, _ = _inputs(dev, rows, dim, "bf16", "f32", False, seed=240)
    ref_dh, ref_dw = _run(dev, h, dy, w, None, rows, dim, "bf16", "f32", "bf16", noalloc=False)
    got_dh, got_dw = _run(dev, h, dy, w, None, rows, dim, "bf16", "f32", "bf16", noalloc=True)
    assert torch.equal(got_dh, ref_dh) and torch.equal(got_dw, ref_dw)
    rows = 513
    h, dy, w, _ = _inputs(dev, rows, dim, "bf16", "f32", False, seed=250)
    dh = torch.full((rows, dim), float("nan"), dtype=torch.bfloat16, device=dev)
    dw = torch.full((dim,), float("nan"), dtype=torch.float32, device=dev)
    rc = _hip.lib().ferrite_hip_rmsnorm_bwd_noalloc(h.data_ptr(), w.data_ptr(), dy.data_ptr(), None, dh.data_ptr(),
                                                    dw.data_ptr(), rows, dim, _hip.BF16, _hip.F32, _hip.BF16, 1e-6,
                                                    _hip.stream_of(h))
    assert rc == 1 and "scratch" in _hip.last_error() and str((512 * dim + rows) * 4) in _hip.last_error()
    torch.cuda.synchronize()
    assert torch.isnan(dw).all() and torch.isnan(dh.float()).all()
