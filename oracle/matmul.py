"""Blocked matmul oracle (test oracle; see oracle/__init__.py).

reference        matmul_reference (matmul.py:129-131): the product with f32 (here
                 f64 for pinning) accumulation, cast to the output dtype.
blocked_padded   the Pallas kernel's algorithm (matmul.py:27-38, :52-86): zero-pad
                 x and y to the block grid, accumulate per (i, j) block over the
                 K blocks in f32, cast on the last step, slice back.
"""

from __future__ import annotations

import numpy as np

from oracle.bf16 import round_bf16


def round_up(x: int, m: int) -> int:
    return -(-x // m) * m


def reference(x, y, *, out_bf16: bool = False, acc=np.float64):
    out = np.asarray(x, acc) @ np.asarray(y, acc)
    out = out.astype(np.float32)
    return round_bf16(out) if out_bf16 else out


def blocked_padded(x, y, *, bm: int, bn: int, bk: int, out_bf16: bool = False):
    x = np.asarray(x, np.float32)
    y = np.asarray(y, np.float32)
    m, k = x.shape
    n = y.shape[1]
    mp, np_, kp = round_up(m, bm), round_up(n, bn), round_up(k, bk)
    xp = np.zeros((mp, kp), np.float32)
    yp = np.zeros((kp, np_), np.float32)
    xp[:m, :k] = x
    yp[:k, :n] = y
    out = np.empty((mp, np_), np.float32)
    for i in range(mp // bm):
        for j in range(np_ // bn):
            acc = np.zeros((bm, bn), np.float32)
            for kk in range(kp // bk):
                acc += xp[i * bm:(i + 1) * bm, kk * bk:(kk + 1) * bk] @ yp[kk * bk:(kk + 1) * bk, j * bn:(j + 1) * bn]
            out[i * bm:(i + 1) * bm, j * bn:(j + 1) * bn] = acc
    out = out[:m, :n]
    return round_bf16(out) if out_bf16 else out
