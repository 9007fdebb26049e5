"""bfloat16 rounding in numpy (test oracle; see oracle/__init__.py).

The reference casts f32 values to bf16 with `astype(jnp.bfloat16)` (e.g.
rmsnorm.py:54, :56; flash_attention.py:114, :126), which is IEEE
round-to-nearest-even on the upper 16 bits. Values are carried as float32
arrays that hold exactly representable bf16 numbers; `bits` gives the uint16
encoding.
"""

from __future__ import annotations

import numpy as np


def round_bf16(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, (x.view(np.uint32) | 0x00400000) & 0xFFFF0000, r).astype(np.uint32)
    return r.view(np.float32)


def bits(x) -> np.ndarray:
    """uint16 bf16 encoding of values that are already bf16-representable."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def from_bits(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)
