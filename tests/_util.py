"""Shared helpers for the tests: seeded inputs and comparisons."""

from __future__ import annotations

import numpy as np
import torch

from oracle.bf16 import round_bf16

TORCH = {"bf16": torch.bfloat16, "f32": torch.float32}


def normal(seed: int, shape, dtype: str = "f32", scale: float = 1.0, loc: float = 0.0) -> np.ndarray:
    """Seeded N(loc, scale^2) values as float32, rounded to bf16 when dtype == 'bf16'."""
    x = (loc + scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)
    return round_bf16(x) if dtype == "bf16" else x


def uniform(seed: int, shape, dtype: str = "f32", lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    x = np.random.default_rng(seed).uniform(lo, hi, shape).astype(np.float32)
    return round_bf16(x) if dtype == "bf16" else x


def to_dev(a: np.ndarray, dtype: str, dev) -> torch.Tensor:
    """Exact transfer: `a` already holds values representable in `dtype`."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(TORCH[dtype])


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) if np.size(a) else 0.0


def rel_fro(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def bf16_ulp(v) -> np.ndarray:
    """Spacing of the bf16 grid at |v| (2^(e-7) for |v| in [2^e, 2^(e+1)))."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.where(a > 0, 2.0 ** (e - 7), 2.0**-133)


def fill_nan(t: torch.Tensor) -> torch.Tensor:
    return t.fill_(float("nan"))
