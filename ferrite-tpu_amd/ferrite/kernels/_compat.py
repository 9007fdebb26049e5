"""Numerics rule and small helpers shared by the kernel wrappers.

Reference: src/ferrite/kernels/_compat.py:17-29. The precision rule is the same:
f32 operands get a true fp32 contraction (fp32 MFMA, v_mfma_f32_32x32x2_f32),
everything else a single bf16 pass (v_mfma_f32_32x32x16_bf16) with f32
accumulation. On MI355X the rule is fixed by the kernel instantiation, so it
does not depend on any process-wide setting.
"""

from __future__ import annotations

import numpy as np
import torch

HIGHEST = "highest"
DEFAULT = "default"

_NAMES = {
    "float32": torch.float32,
    "f32": torch.float32,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
    "float16": torch.float16,
    "float64": torch.float64,
}


def dot_precision(dtype) -> str:
    """'highest' (true fp32 products) for f32 operands, 'default' (one bf16 pass) otherwise."""
    return HIGHEST if to_torch_dtype(dtype) == torch.float32 else DEFAULT


def round_up(x: int, m: int) -> int:
    return -(-x // m) * m


def to_torch_dtype(dtype) -> torch.dtype:
    """Accept a torch dtype, a dtype name ('float32', 'bfloat16') or a numpy dtype."""
    if isinstance(dtype, torch.dtype):
        return dtype
    if isinstance(dtype, str):
        if dtype in _NAMES:
            return _NAMES[dtype]
        raise ValueError(f"unknown dtype name {dtype!r}")
    name = getattr(dtype, "name", None) or np.dtype(dtype).name
    return _NAMES[name]


def dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).replace("torch.", "")
