"""Fused residual-add + RMSNorm oracle (test oracle; see oracle/__init__.py).

Follows src/ferrite/kernels/rmsnorm.py:
  :52-56   h = f32(x) + f32(r); store cast(h); y = h * inv * f32(w) from the
           unrounded f32 h
  :39-43   inv = rsqrt(sum(h*h) * (1/true_dim) + eps), statistics in f32
  :193-199 rmsnorm_reference: the same math
Inputs are float32 arrays holding the storage values (bf16 inputs are passed as
their exact f32 values); `out_bf16` rounds the outputs as the storage cast does.
"""

from __future__ import annotations

import numpy as np

from oracle.bf16 import round_bf16


def add_rmsnorm(x, w, residual=None, *, eps: float = 1e-6, out_bf16: bool = False, acc=np.float32):
    """Return (h, y) with a residual, else y. `acc` is the statistics dtype (float32 as in
    the reference; float64 gives the exact-arithmetic value for pinning)."""
    x = np.asarray(x, dtype=np.float32)
    h32 = x if residual is None else x + np.asarray(residual, dtype=np.float32)  # f32 add, RNE
    h = h32.astype(acc)
    dim = h.shape[-1]
    ss = np.sum(h * h, axis=-1, keepdims=True, dtype=acc)
    inv = 1.0 / np.sqrt(ss * acc(1.0 / dim) + acc(eps))
    y = (h * inv) * np.asarray(w, dtype=acc)
    y = y.astype(np.float32)
    if out_bf16:
        y = round_bf16(y)
        h_out = round_bf16(h32)
    else:
        h_out = h32
    if residual is None:
        return y
    return h_out, y


def rmsnorm_bwd(h, w, dy, eps: float = 1e-6):
    """Analytic backward in float64 (rmsnorm.py:159-166): returns (dh, dw)."""
    h = np.asarray(h, np.float64)
    w = np.asarray(w, np.float64)
    dy = np.asarray(dy, np.float64)
    inv = 1.0 / np.sqrt(np.mean(h * h, axis=-1, keepdims=True) + eps)
    xhat = h * inv
    dw = np.sum(dy * xhat, axis=0)
    dxhat = dy * w
    dh = inv * (dxhat - xhat * np.mean(dxhat * xhat, axis=-1, keepdims=True))
    return dh, dw
