"""Softmax cross-entropy over f32 logits on MI355X HIP kernels.

Reference: src/ferrite/model/gpt.py:147-152 (loss_fn: f32 log_softmax, target
log-likelihood, mean) and its autodiff backward. The forward kernel
(csrc/loss.hip: ferrite_hip_cross_entropy_fwd) reads the logits once and
returns per-row loss and logsumexp; the backward kernel writes
(softmax - onehot) * dloss / N straight into the dtype the caller needs.
"""

from __future__ import annotations

import torch

from ferrite import _hip


def cross_entropy_rows(logits: torch.Tensor, targets: torch.Tensor):
    """(loss, lse), both f32 [N], for f32 logits [N, V] and integer targets [N]."""
    if logits.ndim != 2 or targets.shape != logits.shape[:1]:
        raise ValueError(f"expected logits [N, V] and targets [N]; got {tuple(logits.shape)} and {tuple(targets.shape)}")
    if logits.dtype != torch.float32:
        raise ValueError("logits must be float32")
    _hip.require_gpu(logits, targets)
    logits = logits.contiguous()
    targets = targets.to(torch.int64).contiguous()
    n, v = logits.shape
    loss = torch.empty((n,), dtype=torch.float32, device=logits.device)
    lse = torch.empty((n,), dtype=torch.float32, device=logits.device)
    rc = _hip.lib().ferrite_hip_cross_entropy_fwd(logits.data_ptr(), targets.data_ptr(), loss.data_ptr(),
                                                  lse.data_ptr(), n, v, _hip.stream_of(logits))
    _hip.check(rc, "ferrite_cross_entropy_fwd")
    return loss, lse


def cross_entropy_grad(logits, targets, lse, dloss, scale: float, dtype=torch.float32):
    """d(scale * sum(loss)) / d logits times the 0-d device tensor ``dloss``, in ``dtype``."""
    _hip.require_gpu(logits, targets, lse, dloss)
    logits = logits.contiguous()
    targets = targets.to(torch.int64).contiguous()
    dloss = dloss.to(torch.float32).contiguous()
    n, v = logits.shape
    grad = torch.empty((n, v), dtype=dtype, device=logits.device)
    rc = _hip.lib().ferrite_hip_cross_entropy_bwd(logits.data_ptr(), targets.data_ptr(), lse.data_ptr(),
                                                  dloss.data_ptr(), float(scale), grad.data_ptr(), n, v,
                                                  _hip.dtype_code(dtype), _hip.stream_of(logits))
    _hip.check(rc, "ferrite_cross_entropy_bwd")
    return grad


class _CrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, targets):
        loss, lse = cross_entropy_rows(logits, targets)
        ctx.save_for_backward(logits, targets, lse)
        return loss.mean()

    @staticmethod
    def backward(ctx, dloss):
        logits, targets, lse = ctx.saved_tensors
        return cross_entropy_grad(logits, targets, lse, dloss, 1.0 / logits.shape[0], logits.dtype), None


def cross_entropy(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """Mean softmax cross-entropy of f32 logits [N, V] against targets [N] (differentiable)."""
    return _CrossEntropy.apply(logits, targets)
