"""Fused residual-add + RMSNorm on an MI355X HIP kernel, with a custom VJP.

Reference: src/ferrite/kernels/rmsnorm.py. Same public API and ValueErrors.
The forward is one HIP kernel (csrc/rmsnorm.hip: ferrite_hip_add_rmsnorm /
ferrite_hip_rmsnorm) that reads x and residual once, writes h and y once and
keeps the statistics in f32. As in the reference (rmsnorm.py:9-12, :159-166),
the backward is plain tensor math in f32, here torch ops on the same device.
"""

from __future__ import annotations

import torch

from ferrite import _hip, platform
from ferrite.kernels._compat import round_up

_TARGET_BLOCK_BYTES = 4 << 20


def _rows_block(n_rows: int, dim: int, block_rows: int | None) -> int:
    """Row block of the reference (rmsnorm.py:67-74): validated identically, used only as a hint."""
    if block_rows is None:
        fit = max(platform.SUBLANES, _TARGET_BLOCK_BYTES // (dim * 20))
        fit = 1 << (fit.bit_length() - 1)
        block_rows = min(256, fit, round_up(n_rows, platform.SUBLANES))
    if block_rows % platform.SUBLANES:
        raise ValueError(f"block_rows must be a multiple of {platform.SUBLANES}")
    return block_rows


def _kernel(x2d, r2d, w, eps: float, block_rows):
    """Run the HIP kernel on 2-D x (and residual). Returns y, or (h, y) with a residual."""
    _rows_block(x2d.shape[0], round_up(x2d.shape[1], platform.LANES), block_rows)
    tensors = [x2d, w] if r2d is None else [x2d, r2d, w]
    _hip.require_gpu(*tensors)
    out_dtype = x2d.dtype
    # f32(x) + f32(r): when x and residual differ in dtype, widening the narrower one to f32 first is exact.
    work = out_dtype if r2d is None or r2d.dtype == out_dtype else torch.float32
    x2d = x2d.to(work).contiguous()
    w = w.contiguous()
    rows, dim = x2d.shape
    y = torch.empty_like(x2d)
    lib = _hip.lib()
    stream = _hip.stream_of(x2d)
    if r2d is None:
        rc = lib.ferrite_hip_rmsnorm(
            x2d.data_ptr(), w.data_ptr(), y.data_ptr(), rows, dim, _hip.dtype_code(work), _hip.dtype_code(w.dtype),
            float(eps), stream,
        )
        _hip.check(rc, "ferrite_rmsnorm")
        return y.to(out_dtype)
    r2d = r2d.to(work).contiguous()
    h = torch.empty_like(x2d)
    rc = lib.ferrite_hip_add_rmsnorm(
        x2d.data_ptr(), r2d.data_ptr(), w.data_ptr(), h.data_ptr(), y.data_ptr(), rows, dim,
        _hip.dtype_code(work), _hip.dtype_code(w.dtype), float(eps), stream,
    )
    _hip.check(rc, "ferrite_add_rmsnorm")
    return h.to(out_dtype), y.to(out_dtype)


def _rmsnorm_bwd_math(h, w, dy, eps):
    """Analytic RMSNorm backward in f32 (rmsnorm.py:159-166). y = h * inv * w, inv = rsqrt(mean(h^2) + eps)."""
    inv = torch.rsqrt(torch.mean(h * h, dim=-1, keepdim=True) + eps)
    xhat = h * inv
    dw = torch.sum(dy * xhat, dim=0)
    dxhat = dy * w
    dh = inv * (dxhat - xhat * torch.mean(dxhat * xhat, dim=-1, keepdim=True))
    return dh, dw


class _Norm(torch.autograd.Function):
    """`_norm` of the reference (rmsnorm.py:118-134): residuals (x, w)."""

    @staticmethod
    def forward(ctx, x2d, w, eps, block_rows):
        y = _kernel(x2d, None, w, eps, block_rows)
        ctx.save_for_backward(x2d, w)
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, dy):
        x2d, w = ctx.saved_tensors
        dx, dw = _rmsnorm_bwd_math(x2d.float(), w.float(), dy.float(), ctx.eps)
        return dx.to(x2d.dtype), dw.to(w.dtype), None, None


class _AddNorm(torch.autograd.Function):
    """`_add_norm` of the reference (rmsnorm.py:137-156): residuals (rounded h, w); bwd returns (dh, dh, dw)."""

    @staticmethod
    def forward(ctx, x2d, r2d, w, eps, block_rows):
        h, y = _kernel(x2d, r2d, w, eps, block_rows)
        ctx.save_for_backward(h, w)
        ctx.eps = eps
        ctx.r_dtype = r2d.dtype
        return h, y

    @staticmethod
    def backward(ctx, dh_direct, dy):
        h, w = ctx.saved_tensors
        dh, dw = _rmsnorm_bwd_math(h.float(), w.float(), dy.float(), ctx.eps)
        dh = dh + dh_direct.float()
        return dh.to(h.dtype), dh.to(ctx.r_dtype), dw.to(w.dtype), None, None


def rmsnorm(x, weight, *, residual=None, eps: float = 1e-6, block_rows: int | None = None):
    """RMSNorm over the last axis of ``x`` (rmsnorm.py:174-190).

    With ``residual`` given, returns ``(h, y)`` where ``h = x + residual`` is the
    new residual stream and ``y = rmsnorm(h) * weight``; otherwise returns ``y``.
    """
    dim = x.shape[-1]
    if tuple(weight.shape) != (dim,):
        raise ValueError(f"weight must have shape ({dim},), got {tuple(weight.shape)}")
    lead = x.shape[:-1]
    x2d = x.reshape(-1, dim)
    if residual is None:
        return _Norm.apply(x2d, weight, float(eps), block_rows).reshape(*lead, dim)
    if residual.shape != x.shape:
        raise ValueError("residual must match x")
    h, y = _AddNorm.apply(x2d, residual.reshape(-1, dim), weight, float(eps), block_rows)
    return h.reshape(*lead, dim), y.reshape(*lead, dim)


def rmsnorm_reference(x, weight, *, residual=None, eps: float = 1e-6):
    """Plain torch math with identical f32 numerics (the reference's XLA route, rmsnorm.py:193-199)."""
    h = x.float() + (0 if residual is None else residual.float())
    y = h * torch.rsqrt(torch.mean(h * h, dim=-1, keepdim=True) + eps) * weight.float()
    if residual is None:
        return y.to(x.dtype)
    return h.to(x.dtype), y.to(x.dtype)
