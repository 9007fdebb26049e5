"""CPU tests of the boundary: the C ABI library loads and exports every symbol
of include/ferrite_hip.h, its argument checks return error codes without
touching a GPU, and the Python API raises the reference's ValueErrors before
dispatch and refuses (loudly) to run on CPU tensors."""

import os
import re
import subprocess

import pytest
import torch

from ferrite import _hip, platform
from ferrite.kernels import (BlockSizes, attention_flops, flash_attention, flash_attention_reference, matmul,
                             matmul_flops, matmul_reference, rmsnorm, rmsnorm_reference)
from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ferrite_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(ferrite_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    declared = _declared_symbols()
    assert len(declared) == 36
    out = subprocess.run(["nm", "-D", "--defined-only", _hip.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(\w+)", out))
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    assert set(declared) == set(_hip.SIGNATURES)
    for s in declared:
        getattr(_hip.lib(), s)


def test_abi_argument_checks_return_codes():
    lib = _hip.lib()
    assert lib.ferrite_hip_version().startswith(b"ferrite_hip")
    assert lib.ferrite_hip_matmul(None, None, None, 0, 4, 4, _hip.BF16, _hip.BF16, None) == 1
    assert "M, N, K" in _hip.last_error()
    assert lib.ferrite_hip_matmul(None, None, None, 4, 4, 4, 7, _hip.BF16, None) == 1
    assert "dtype" in _hip.last_error()
    # RMSNorm backward: workspace query, dtype, shape and null-pointer checks
    assert lib.ferrite_hip_rmsnorm_bwd_workspace(8192, 768) == (512 * 768 + 8192) * 4
    assert lib.ferrite_hip_rmsnorm_bwd_workspace(-1, 768) == -1
    assert lib.ferrite_hip_rmsnorm_bwd(1, 1, 1, None, 1, 1, 1, 4, 8, _hip.BF16, 5, _hip.BF16, 1e-6, None) == 1
    assert "dtype" in _hip.last_error()
    assert lib.ferrite_hip_rmsnorm_bwd(1, 1, 1, None, 1, 1, 1, 4, 0, _hip.BF16, _hip.F32, _hip.BF16, 1e-6, None) == 1
    assert lib.ferrite_hip_rmsnorm_bwd(1, 1, None, None, 1, 1, 1, 4, 8, _hip.BF16, _hip.F32, _hip.BF16, 1e-6, None) == 1
    assert "null" in _hip.last_error()
    assert lib.ferrite_hip_rmsnorm_bwd(1, 1, 1, None, 1, 1, 1, 4, 8, _hip.F32, _hip.F32, _hip.BF16, 1e-6, None) == 1
    # the allocation-free backward: shapes beyond its fixed scratch are refused before any device call
    a = 1 << 12  # 16-byte aligned stand-in addresses: the fast path's plan (512 partial rows of dim floats)
    assert lib.ferrite_hip_rmsnorm_bwd_noalloc(a, a, a, None, a, a, 1 << 20, 8192, _hip.BF16, _hip.F32, _hip.BF16,
                                               1e-6, None) == 1
    assert "scratch" in _hip.last_error() and str(_hip.RMSNORM_BWD_SCRATCH_BYTES) in _hip.last_error()
    assert lib.ferrite_hip_rmsnorm_bwd_noalloc(a, a, a, None, a, a, 16, 8, _hip.BF16, 9, _hip.BF16, 1e-6, None) == 1
    assert "dtype" in _hip.last_error()
    assert lib.ferrite_hip_rmsnorm_bwd_noalloc(a, a, None, None, a, a, 16, 8, _hip.BF16, _hip.F32, _hip.BF16, 1e-6,
                                               None) == 1
    assert "null" in _hip.last_error()
    # AdamW: workspace query and argument checks (host arrays are inspected before any launch)
    assert lib.ferrite_hip_adamw_workspace(75) == (3 * 2048 + 4) * 4
    assert lib.ferrite_hip_adamw_workspace(-1) == -1
    args = [None] * 6 + [_hip.BF16, _hip.BF16, 1e-3, 0.9, 0.95, 1e-8, 0.1, 1.0]
    assert lib.ferrite_hip_adamw(1, *args, 1, None, None, 1, None) == 1
    assert "null" in _hip.last_error()
    assert lib.ferrite_hip_adamw(0, *args, 0, None, None, 1, None) == 1
    assert "step" in _hip.last_error()
    assert lib.ferrite_hip_adamw(0, *args[:6], 9, _hip.BF16, *args[8:], 1, None, None, 1, None) == 1
    # head layout: group count, dtype and null checks; empty is a no-op
    assert lib.ferrite_hip_heads_split(None, None, 0, 4, 3, 2, 8, _hip.BF16, None) == 0
    assert lib.ferrite_hip_heads_split(1, 1, 2, 4, 5, 2, 8, _hip.BF16, None) == 1
    assert lib.ferrite_hip_heads_merge(1, 1, 2, 4, 3, 2, 8, 4, None) == 1
    assert lib.ferrite_hip_heads_merge(None, 1, 2, 4, 3, 2, 8, _hip.BF16, None) == 1
    assert "null" in _hip.last_error()
    # cross-entropy: shape, dtype and null checks; n == 0 is a no-op
    assert lib.ferrite_hip_cross_entropy_fwd(None, None, None, None, 0, 8, None) == 0
    assert lib.ferrite_hip_cross_entropy_fwd(1, 1, 1, 1, 4, 0, None) == 1
    assert lib.ferrite_hip_cross_entropy_fwd(None, 1, 1, 1, 4, 8, None) == 1
    assert "null" in _hip.last_error()
    assert lib.ferrite_hip_cross_entropy_bwd(1, 1, 1, 1, 1.0, 1, 4, 8, 3, None) == 1
    assert lib.ferrite_hip_cross_entropy_bwd(1, 1, 1, None, 1.0, 1, 4, 8, _hip.BF16, None) == 1
    # causal needs sq == sk
    assert lib.ferrite_hip_attn_fwd(1, 1, 1, 1, 1, 1, 1, 128, 256, 64, _hip.BF16, 1, 0.125, None) == 1
    assert "sq == sk" in _hip.last_error()
    # head dims the reference refuses (above 128 and not a multiple of 128) are refused here too;
    # every multiple of 128 is taken, forward and backward (flash_attention.py:341-343)
    for d in (200, 320, 136):
        assert lib.ferrite_hip_attn_fwd(1, 1, 1, 1, 1, 1, 1, 128, 128, d, _hip.BF16, 1, 0.1, None) == 1
        assert "multiple of 128" in _hip.last_error()
        assert lib.ferrite_hip_attn_bwd_dq(1, 1, 1, 1, 1, 1, 1, 1, 1, 128, 128, d, _hip.BF16, 1, 0.1, None) == 1
        assert lib.ferrite_hip_attn_bwd_dkv(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 128, 128, d, _hip.BF16, 1, 0.1, None) == 1
        assert "multiple of 128" in _hip.last_error()
    assert lib.ferrite_hip_add_rmsnorm(None, None, None, None, None, 4, 0, 1, 1, 1e-6, None) == 1
    # the streaming copy: size and alignment checks; zero bytes is a no-op
    assert lib.ferrite_hip_stream_copy2(None, None, None, None, 0, None) == 0
    assert lib.ferrite_hip_stream_copy2(16, 16, 16, 16, 24, None) == 1 and "multiple of 16" in _hip.last_error()
    assert lib.ferrite_hip_stream_copy2(16, 8, 16, 16, 32, None) == 1 and "unaligned" in _hip.last_error()
    # rows == 0 is a valid no-op and launches nothing
    assert lib.ferrite_hip_rmsnorm(None, None, None, 0, 16, 1, 1, 1e-6, None) == 0


def _qkv(s=256, d=128, dtype=torch.float32):
    g = torch.Generator().manual_seed(0)
    return tuple(torch.randn(1, 1, s, d, generator=g).to(dtype) for _ in range(3))


def test_flash_attention_validation_errors():
    """Mirrors the reference's test_validation_errors (tests/test_flash_attention.py:69-76)."""
    q, k, v = _qkv()
    with pytest.raises(ValueError):
        flash_attention(q, k, v, block_sizes=BlockSizes(block_k=100))
    with pytest.raises(ValueError):
        flash_attention(q, k[:, :, :128], v[:, :, :128], causal=True)
    with pytest.raises(ValueError):
        flash_attention(q, k, v.to(torch.bfloat16))
    with pytest.raises(ValueError):
        flash_attention(q[..., :1], k, v)  # mismatched head dims
    qq = torch.zeros(1, 1, 256, 200)
    with pytest.raises(ValueError):  # d > 128 and not a multiple of 128
        flash_attention(qq, qq, qq)
    with pytest.raises(ValueError):
        flash_attention(q, k, v, block_sizes=BlockSizes(block_q=12))


def test_matmul_and_rmsnorm_validation_errors():
    x = torch.zeros(128, 128)
    with pytest.raises(ValueError):
        matmul(x, x, block_n=100)
    with pytest.raises(ValueError):
        matmul(x, torch.zeros(64, 128))
    with pytest.raises(ValueError):
        rmsnorm(x, torch.ones(64))
    with pytest.raises(ValueError):
        rmsnorm(x, torch.ones(128), residual=torch.zeros(64, 128))
    with pytest.raises(ValueError):
        rmsnorm(x, torch.ones(128), block_rows=12)


def test_product_path_refuses_cpu_tensors():
    q, k, v = _qkv()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        flash_attention(q, k, v)
    x = torch.zeros(128, 128)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        matmul(x, x)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        rmsnorm(x, torch.ones(128))


def test_reference_functions_and_flop_formulas():
    q, k, v = _qkv(s=16, d=8)
    out = flash_attention_reference(q, k, v, causal=True)
    torch.testing.assert_close(out[:, :, 0], v[:, :, 0])
    assert attention_flops(4, 16, 2048, 2048, 128, causal=True) == 68_719_476_736
    assert attention_flops(4, 16, 2048, 2048, 128, causal=True, backward=True) == int(68_719_476_736 * 2.5)
    assert matmul_flops(4096, 4096, 4096) == 2 * 4096**3
    x = torch.randn(4, 8)
    torch.testing.assert_close(matmul_reference(x, torch.eye(8)), x)
    h, y = rmsnorm_reference(x, torch.ones(8), residual=x)
    torch.testing.assert_close(h, 2 * x)


def test_platform_peaks():
    p = platform.peaks("MI355X")
    assert p.bf16_flops == pytest.approx(2.5166e15) and p.hbm_bytes_per_s == 8e12
    assert p.ridge_point > 300
    assert BlockSizes.for_device() == BlockSizes(128, 128, 128, 128)
    with platform.interpret_mode() as on:
        assert on is False


def test_stream_kernels_argument_checks():
    """Bad sizes, grids and pointers are refused before any launch (runs on the CPU path too)."""
    lib = _hip.lib()
    assert lib.ferrite_hip_stream_read(None, 15, None, 0, None) == 1
    assert "multiple of 16" in _hip.last_error()
    assert lib.ferrite_hip_stream_read(None, 16, None, 70000, None) == 1
    assert "blocks" in _hip.last_error()
    assert lib.ferrite_hip_stream_fill(None, 32, 1, 0, None) == 1
    assert "null" in _hip.last_error()
    assert lib.ferrite_hip_stream_fill(None, 0, 1, 0, None) == 0
    assert lib.ferrite_hip_mfma_ceiling(None, 256, 8, 16, None) == 1
    assert "sink" in _hip.last_error()
    assert lib.ferrite_hip_mfma_ceiling(None, 256, 6, 16, None) == 1
    assert "waves 4 or 8" in _hip.last_error()
    assert lib.ferrite_hip_mfma_ceiling(None, 0, 8, 16, None) == 1


def test_forward_workspace_query():
    """ferrite_hip_attn_fwd_workspace: the split long-context forward's workspace for the shapes it
    takes (bf16, causal, d <= 64, an even number of 128-row tiles, a grid resident at once, at
    least 16 tiles with one workgroup per CU or 64 with two), 0 for every other shape, -1 for
    invalid ones; a positive size with no workspace is refused. (256 CUs: no device here.)"""
    lib = _hip.lib()
    bf, f32 = _hip.BF16, _hip.F32
    per_pair = 2 * (8192 + 256) * 4 + 4
    assert lib.ferrite_hip_attn_fwd_workspace(1, 8, 8192, 8192, 64, bf, 1) == 256 * per_pair
    assert lib.ferrite_hip_attn_fwd_workspace(1, 1, 2048, 2048, 48, bf, 1) == 8 * per_pair
    for args in [(1, 8, 8192, 8192, 128, bf, 1),   # the D = 128 kernel is not split
                 (1, 1, 1792, 1792, 64, bf, 1),    # one workgroup per CU, fewer than 16 query tiles
                 (4, 8, 4096, 4096, 64, bf, 1),    # two per CU, fewer than 64 query tiles
                 (1, 8, 8192, 8192, 64, bf, 0),    # non-causal
                 (1, 8, 8192, 8192, 64, f32, 1),   # f32
                 (1, 8, 8192 - 64, 8192 - 64, 64, bf, 1),  # S not a multiple of 128
                 (1, 1, 1152, 1152, 64, bf, 1),    # an odd number of tiles (9)
                 (8, 12, 1024, 1024, 64, bf, 1),   # more tiles than resident workgroups (the GPT shape)
                 (1, 8, 8192, 4096, 64, bf, 1)]:   # sq != sk
        assert lib.ferrite_hip_attn_fwd_workspace(*args) == 0, args
    assert lib.ferrite_hip_attn_fwd_workspace(0, 8, 8192, 8192, 64, bf, 1) == -1
    rc = lib.ferrite_hip_attn_fwd_ex(1, 1, 1, 1, 1, 1, 8, 8192, 8192, 64, bf, 1, 0.125, None, 1024, None)
    assert rc == 1 and "workspace" in _hip.last_error()


def test_backward_workspace_query():
    """ferrite_hip_attn_bwd_workspace: the split dK/dV and dQ's shared workspace (one 4-byte count
    per pair of 128-row tiles, rounded up to 256 bytes, then two 64 KiB dK+dV shares per pair) for
    the forward's long-context shapes and, with two workgroups per CU, from 32 tiles on (the
    forward splits from 64), 0 elsewhere, -1 for invalid shapes; each _ex entry point refuses a
    positive size with no workspace. (256 CUs: no device here.)"""
    lib = _hip.lib()
    bf, f32 = _hip.BF16, _hip.F32
    assert lib.ferrite_hip_attn_bwd_workspace(1, 8, 8192, 8192, 64, bf, 1) == 1024 + 256 * 2 * 65536
    assert lib.ferrite_hip_attn_bwd_workspace(1, 1, 2048, 2048, 48, bf, 1) == 256 + 8 * 2 * 65536
    assert lib.ferrite_hip_attn_bwd_workspace(1, 4, 8192, 8192, 64, bf, 1) == 512 + 128 * 2 * 65536
    assert lib.ferrite_hip_attn_bwd_workspace(1, 16, 4096, 4096, 64, bf, 1) == 1024 + 256 * 2 * 65536  # 32 tiles, two per CU
    for args in [(1, 8, 8192, 8192, 128, bf, 1), (1, 1, 1792, 1792, 64, bf, 1), (4, 8, 4096, 4096, 64, bf, 1),
                 (4, 8, 2048, 2048, 64, bf, 1), (1, 8, 8192, 8192, 64, bf, 0), (1, 8, 8192, 8192, 64, f32, 1),
                 (1, 8, 8128, 8128, 64, bf, 1),
                 (1, 1, 1152, 1152, 64, bf, 1), (8, 12, 1024, 1024, 64, bf, 1), (1, 8, 8192, 4096, 64, bf, 1),
                 (2, 8, 8192, 8192, 64, bf, 1)]:  # 1024 tiles: not resident at once
        assert lib.ferrite_hip_attn_bwd_workspace(*args) == 0, args
    assert lib.ferrite_hip_attn_bwd_workspace(1, 0, 8192, 8192, 64, bf, 1) == -1
    p = [1] * 8
    rc = lib.ferrite_hip_attn_bwd_dkv_ex(*p, 1, 8, 8192, 8192, 64, bf, 1, 0.125, None, 1024, None)
    assert rc == 1 and "workspace" in _hip.last_error()
    rc = lib.ferrite_hip_attn_bwd_dq_ex(*p[:7], 1, 8, 8192, 8192, 64, bf, 1, 0.125, None, 1024, None)
    assert rc == 1 and "workspace" in _hip.last_error()
    rc = lib.ferrite_hip_attn_bwd_dq_delta_ex(*p, 1, 8, 8192, 8192, 64, bf, 1, 0.125, None, 1024, None)
    assert rc == 1 and "workspace" in _hip.last_error()
