"""Fused residual-add + RMSNorm on an MI355X HIP kernel, with a custom VJP.

Reference: src/ferrite/kernels/rmsnorm.py. Same public API and ValueErrors.
The forward is one HIP kernel (csrc/rmsnorm.hip: ferrite_hip_add_rmsnorm /
ferrite_hip_rmsnorm) that reads x and residual once, writes h and y once and
keeps the statistics in f32. The backward (rmsnorm.py:159-166, an XLA fusion in
the reference) is a HIP kernel too (ferrite_hip_rmsnorm_bwd): one pass over h,
dy and the fused add's direct gradient that writes dh, plus a fixed-order
reduction of dweight.
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


def _bwd_kernel(h2d, w, dy, dd, eps: float, dh_dtype):
    """(dh, dw) of the analytic backward on the HIP kernel; `dd` is the fused add's direct
    gradient (or None). dh comes back in `dh_dtype` (h's dtype or float32), dw in w's dtype."""
    _hip.require_gpu(h2d, w, dy)
    h2d, dy, w = h2d.contiguous(), dy.to(h2d.dtype).contiguous(), w.contiguous()
    if dd is not None:
        dd = dd.to(h2d.dtype).contiguous()
    rows, dim = h2d.shape
    lib = _hip.lib()
    dh = torch.empty((rows, dim), dtype=dh_dtype, device=h2d.device)
    dw = torch.empty_like(w)
    ws = torch.empty((lib.ferrite_hip_rmsnorm_bwd_workspace(rows, dim) + 3) // 4, dtype=torch.float32, device=h2d.device)
    rc = lib.ferrite_hip_rmsnorm_bwd(
        h2d.data_ptr(), w.data_ptr(), dy.data_ptr(), _hip.ptr(dd), dh.data_ptr(), dw.data_ptr(), ws.data_ptr(),
        rows, dim, _hip.dtype_code(h2d.dtype), _hip.dtype_code(w.dtype), _hip.dtype_code(dh_dtype), float(eps),
        _hip.stream_of(h2d),
    )
    _hip.check(rc, "ferrite_rmsnorm_bwd")
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
        dx, dw = _bwd_kernel(x2d, w, dy, None, ctx.eps, x2d.dtype)
        return dx, dw, None, None


class _AddNorm(torch.autograd.Function):
    """`_add_norm` of the reference (rmsnorm.py:137-156): residuals (rounded h, w); bwd returns (dh, dh, dw)."""

    @staticmethod
    def forward(ctx, x2d, r2d, w, eps, block_rows):
        h, y = _kernel(x2d, r2d, w, eps, block_rows)
        ctx.save_for_backward(h, w)
        ctx.eps = eps
        ctx.r_dtype = r2d.dtype
        ctx.set_materialize_grads(False)  # an unused h (the last norm's) costs no zero tensor
        return h, y

    @staticmethod
    def backward(ctx, dh_direct, dy):
        h, w = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(h)
        # dh in h's dtype serves both inputs when the residual has it too; otherwise keep f32
        # and round once per input, as the reference's casts of the f32 dh do.
        same = ctx.r_dtype == h.dtype
        dh, dw = _bwd_kernel(h, w, dy, dh_direct, ctx.eps, h.dtype if same else torch.float32)
        if same:
            return dh, dh, dw, None, None
        return dh.to(h.dtype), dh.to(ctx.r_dtype), dw, None, None


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
