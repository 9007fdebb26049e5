"""Flash attention oracle (test oracle; see oracle/__init__.py).

Layout q, k, v, dO: [B, H, S, D] float arrays holding the storage values.

forward          flash_attention_reference (flash_attention.py:370-380): f32 (or
                 f64) scores * scale, tril(k = sk - sq) mask with the finite
                 MASK_VALUE, softmax, P @ V; plus the logsumexp of the visible
                 scaled scores (the `lse` the kernels save, :127).
backward         FA-2 analytic gradients (:184-243, :326-330): P from the scores,
                 delta = rowsum(dO * O), dV = P^T dO, dP = dO V^T,
                 dS = P * (dP - delta), dQ = scale dS K, dK = scale dS^T Q.
flash_forward    the Pallas forward kernel's own algorithm (:91-127): per
                 (q block, kv block) online softmax in f32 with block skipping,
                 P cast to the input dtype before P @ V, O = acc * (1/l),
                 lse = m + log(l).
flash_backward   the Pallas dK/dV and dQ kernels (:184-243): P = exp(S - lse),
                 dS = P * (dP - delta), P and dS cast to the input dtype before
                 the products, dK and dQ scaled at the end.
"""

from __future__ import annotations

import math

import numpy as np

from oracle.bf16 import round_bf16

MASK_VALUE = -0.7 * float(np.finfo(np.float32).max)


def _scale(d: int, scale):
    return 1.0 / math.sqrt(d) if scale is None else float(scale)


def _mask(sq: int, sk: int) -> np.ndarray:
    return np.tril(np.ones((sq, sk), dtype=bool), k=sk - sq)


def forward(q, k, v, *, causal: bool = True, scale=None, dtype=np.float64):
    """Materialised attention. Returns (O, lse) in `dtype`."""
    q, k, v = (np.asarray(a, dtype=dtype) for a in (q, k, v))
    b, h, sq, d = q.shape
    sk = k.shape[2]
    sc = dtype(_scale(d, scale))
    o = np.empty((b, h, sq, d), dtype=dtype)
    lse = np.empty((b, h, sq), dtype=dtype)
    mask = _mask(sq, sk) if causal else None
    for bi in range(b):
        for hi in range(h):
            s = (q[bi, hi] @ k[bi, hi].T) * sc
            if causal:
                s = np.where(mask, s, dtype(MASK_VALUE))
            m = s.max(axis=-1, keepdims=True)
            e = np.exp(s - m)
            l = e.sum(axis=-1, keepdims=True)
            o[bi, hi] = (e / l) @ v[bi, hi]
            lse[bi, hi] = (m + np.log(l))[:, 0]
    return o, lse


def backward(q, k, v, do, *, causal: bool = True, scale=None, dtype=np.float64):
    """FA-2 analytic gradients in `dtype` (float64 by default). Returns (dq, dk, dv)."""
    q, k, v, do = (np.asarray(a, dtype=dtype) for a in (q, k, v, do))
    b, h, sq, d = q.shape
    sk = k.shape[2]
    sc = dtype(_scale(d, scale))
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    mask = _mask(sq, sk) if causal else None
    for bi in range(b):
        for hi in range(h):
            s = (q[bi, hi] @ k[bi, hi].T) * sc
            if causal:
                s = np.where(mask, s, dtype(MASK_VALUE))
            p = np.exp(s - s.max(axis=-1, keepdims=True))
            p /= p.sum(axis=-1, keepdims=True)
            o = p @ v[bi, hi]
            delta = np.sum(do[bi, hi] * o, axis=-1, keepdims=True)
            dv[bi, hi] = p.T @ do[bi, hi]
            dp = do[bi, hi] @ v[bi, hi].T
            ds = p * (dp - delta)
            dq[bi, hi] = sc * (ds @ k[bi, hi])
            dk[bi, hi] = sc * (ds.T @ q[bi, hi])
    return dq, dk, dv


def _cast(x, bf16: bool):
    return round_bf16(x) if bf16 else np.asarray(x, np.float32)


def flash_forward(q, k, v, *, causal: bool = True, scale=None, bq: int = 128, bk: int = 128, bf16: bool = False):
    """The reference's blockwise forward kernel in f32. Returns (O, lse) as float32
    (O rounded to bf16 when `bf16`)."""
    q, k, v = (np.asarray(a, dtype=np.float32) for a in (q, k, v))
    b, h, sq, d = q.shape
    sk = k.shape[2]
    sc = np.float32(_scale(d, scale))
    o = np.empty((b, h, sq, d), np.float32)
    lse = np.empty((b, h, sq), np.float32)
    for bi in range(b):
        for hi in range(h):
            for qi in range(sq // bq):
                qb = q[bi, hi, qi * bq:(qi + 1) * bq]
                m = np.full((bq, 1), -np.inf, np.float32)
                l = np.zeros((bq, 1), np.float32)
                acc = np.zeros((bq, d), np.float32)
                for ki in range(sk // bk):
                    if causal and not ((qi + 1) * bq - 1 >= ki * bk):
                        continue
                    kb = k[bi, hi, ki * bk:(ki + 1) * bk]
                    vb = v[bi, hi, ki * bk:(ki + 1) * bk]
                    s = (qb @ kb.T) * sc
                    if causal:
                        rows = qi * bq + np.arange(bq)[:, None]
                        cols = ki * bk + np.arange(bk)[None, :]
                        s = np.where(cols <= rows, s, np.float32(MASK_VALUE))
                    m_next = np.maximum(m, s.max(axis=1, keepdims=True))
                    p = np.exp(s - m_next)
                    alpha = np.exp(m - m_next)
                    l = alpha * l + p.sum(axis=1, keepdims=True)
                    m = m_next
                    acc = acc * alpha + _cast(p, bf16) @ vb
                o[bi, hi, qi * bq:(qi + 1) * bq] = acc * (np.float32(1.0) / l)
                lse[bi, hi, qi * bq:(qi + 1) * bq] = (m + np.log(l))[:, 0]
    return _cast(o, bf16), lse


def flash_backward(q, k, v, do, o, lse, *, causal: bool = True, scale=None, bq: int = 128, bk: int = 128,
                   bf16: bool = False):
    """The reference's dK/dV and dQ kernels in f32. Returns (dq, dk, dv) as float32."""
    q, k, v, do, o = (np.asarray(a, dtype=np.float32) for a in (q, k, v, do, o))
    lse = np.asarray(lse, np.float32)
    b, h, sq, d = q.shape
    sk = k.shape[2]
    sc = np.float32(_scale(d, scale))
    delta = np.sum(do * o, axis=-1)  # f32, :328
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for bi in range(b):
        for hi in range(h):
            for ki in range(sk // bk):
                for qi in range(sq // bq):
                    if causal and not ((qi + 1) * bq - 1 >= ki * bk):
                        continue
                    qs, ks_ = slice(qi * bq, (qi + 1) * bq), slice(ki * bk, (ki + 1) * bk)
                    qb, kb, vb, dob = q[bi, hi, qs], k[bi, hi, ks_], v[bi, hi, ks_], do[bi, hi, qs]
                    s = (qb @ kb.T) * sc
                    if causal:
                        rows = qi * bq + np.arange(bq)[:, None]
                        cols = ki * bk + np.arange(bk)[None, :]
                        s = np.where(cols <= rows, s, np.float32(MASK_VALUE))
                    p = np.exp(s - lse[bi, hi, qs][:, None])
                    dp = dob @ vb.T
                    ds = p * (dp - delta[bi, hi, qs][:, None])
                    dv[bi, hi, ks_] += _cast(p, bf16).T @ dob
                    dk[bi, hi, ks_] += _cast(ds, bf16).T @ qb
                    dq[bi, hi, qs] += _cast(ds, bf16) @ kb
    return _cast(dq * sc, bf16), _cast(dk * sc, bf16), _cast(dv, bf16)


def brute_force(q, k, v, *, causal: bool = True, scale=None):
    """Pure-Python definition O_i = sum_j softmax_j(scale q_i.k_j) v_j, lse_i = log sum_j exp(...),
    over the visible keys only. For tiny inputs; used to pin `forward`."""
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    b, h, sq, d = q.shape
    sk = k.shape[2]
    sc = _scale(d, scale)
    o = np.zeros((b, h, sq, d))
    lse = np.zeros((b, h, sq))
    for bi in range(b):
        for hi in range(h):
            for i in range(sq):
                js = [j for j in range(sk) if not causal or j <= i + (sk - sq)]
                scores = [sc * sum(q[bi, hi, i, t] * k[bi, hi, j, t] for t in range(d)) for j in js]
                mx = max(scores)
                ws = [math.exp(s - mx) for s in scores]
                tot = sum(ws)
                lse[bi, hi, i] = mx + math.log(tot)
                for c in range(d):
                    o[bi, hi, i, c] = sum(w * v[bi, hi, j, c] for w, j in zip(ws, js)) / tot
    return o, lse
