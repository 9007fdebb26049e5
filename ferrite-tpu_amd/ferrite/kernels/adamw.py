"""Fused AdamW step on an MI355X HIP kernel.

Reference: src/ferrite/model/train.py:59-74 (adamw_update), which XLA fuses
over the parameter tree. Here one call (csrc/optim.hip: ferrite_hip_adamw)
computes the global gradient norm, the clip scale and the update of every
tensor with three kernels and no host synchronisation; each element of
g, p, m and v is read once and p, m, v written once.
"""

from __future__ import annotations

import ctypes

import torch

from ferrite import _hip


def _ptrs(tensors) -> ctypes.c_void_p:
    arr = (ctypes.c_void_p * max(1, len(tensors)))(*[t.data_ptr() for t in tensors])
    return ctypes.cast(arr, ctypes.c_void_p), arr


def fused_adamw_(params, grads, exp_avg, exp_avg_sq, decay, *, lr: float, beta1: float, beta2: float, eps: float,
                 weight_decay: float, max_grad_norm: float, step: int, step_scalars: torch.Tensor | None = None,
                 grad_norm: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Update ``params``, ``exp_avg`` and ``exp_avg_sq`` in place; return the pre-clip global
    gradient norm as a 0-d f32 device tensor.

    ``params``: same-dtype (f32 or bf16) contiguous device tensors; ``grads``: matching shapes,
    one dtype; moments: f32 like ``params``; ``decay``: per-tensor bools (weight decay on).
    ``step_scalars`` (f32 device tensor [3] = lr, 1 - beta1^step, 1 - beta2^step) replaces
    ``lr`` and ``step`` at run time, for replay inside a captured graph; ``grad_norm`` and
    ``workspace`` may be given to reuse buffers across calls."""
    n = len(params)
    if not (len(grads) == len(exp_avg) == len(exp_avg_sq) == len(decay) == n):
        raise ValueError("params, grads, moments and decay flags must have the same length")
    if n == 0:
        raise ValueError("no tensors")
    _hip.require_gpu(*params, *grads, *exp_avg, *exp_avg_sq)
    pdt, gdt = params[0].dtype, grads[0].dtype
    for p, g, m, v in zip(params, grads, exp_avg, exp_avg_sq):
        if p.dtype != pdt or g.dtype != gdt or m.dtype != torch.float32 or v.dtype != torch.float32:
            raise ValueError("params share one dtype, grads one dtype, moments are float32")
        if not (p.is_contiguous() and m.is_contiguous() and v.is_contiguous()):
            raise ValueError("params and moments must be contiguous (they are updated in place)")
        if g.shape != p.shape or m.shape != p.shape or v.shape != p.shape:
            raise ValueError("grads and moments must match their parameter's shape")
    grads = [g.contiguous() for g in grads]
    lib = _hip.lib()
    dev = params[0].device
    ws_floats = (lib.ferrite_hip_adamw_workspace(n) + 3) // 4
    ws = workspace if workspace is not None and workspace.numel() >= ws_floats else torch.empty(
        (ws_floats,), dtype=torch.float32, device=dev)
    gnorm = grad_norm if grad_norm is not None else torch.empty((), dtype=torch.float32, device=dev)
    if step_scalars is not None and (step_scalars.dtype != torch.float32 or step_scalars.numel() < 3):
        raise ValueError("step_scalars must be a float32 device tensor of 3 values")
    pp, _a = _ptrs(params)
    gp, _b = _ptrs(grads)
    mp, _c = _ptrs(exp_avg)
    vp, _d = _ptrs(exp_avg_sq)
    numel = (ctypes.c_int64 * n)(*[p.numel() for p in params])
    flags = (ctypes.c_int32 * n)(*[1 if f else 0 for f in decay])
    rc = lib.ferrite_hip_adamw(
        n, pp, gp, mp, vp, ctypes.cast(numel, ctypes.c_void_p), ctypes.cast(flags, ctypes.c_void_p),
        _hip.dtype_code(pdt), _hip.dtype_code(gdt), float(lr), float(beta1), float(beta2), float(eps),
        float(weight_decay), float(max_grad_norm), int(step), _hip.ptr(step_scalars), gnorm.data_ptr(), ws.data_ptr(),
        _hip.stream_of(params[0]),
    )
    _hip.check(rc, "ferrite_adamw")
    return gnorm
