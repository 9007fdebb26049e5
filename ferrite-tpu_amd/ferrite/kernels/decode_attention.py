"""Decode attention over a static KV cache on an MI355X HIP kernel.

Reference: src/ferrite/serving/engine.py:89-104 (_cache_attention, _write_cache),
which the reference leaves to XLA; a decode-attention kernel is its own named
next step. One call (csrc/decode.hip: ferrite_hip_decode_attention) writes the
new key/value rows into the cache at each sequence's position and attends the
query over keys 0..pos, split over key chunks (a power of two from 256 keys up,
as few as keep the grid within 512 workgroups) merged in f32.
"""

from __future__ import annotations

import math

import torch

from ferrite import _hip


def decode_attention(q, k_new, v_new, k_cache, v_cache, pos, *, scale: float | None = None):
    """q, k_new, v_new [B, H, D]; caches [B, H, max_len, D] (updated in place at ``pos``);
    pos int32 [B] on the device. Returns [B, H, D] in q's dtype. A position outside
    [0, max_len) writes nothing and yields NaN for that sequence."""
    if q.ndim != 3 or k_new.shape != q.shape or v_new.shape != q.shape:
        raise ValueError(f"expected q, k_new, v_new as [B, H, D]; got {tuple(q.shape)}, {tuple(k_new.shape)}, {tuple(v_new.shape)}")
    b, h, d = q.shape
    if k_cache.ndim != 4 or k_cache.shape[:2] != (b, h) or k_cache.shape[3] != d or v_cache.shape != k_cache.shape:
        raise ValueError(f"expected caches [B, H, max_len, D] matching q; got {tuple(k_cache.shape)}, {tuple(v_cache.shape)}")
    if not (q.dtype == k_new.dtype == v_new.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("q, k_new, v_new and the caches must share a dtype")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("the caches must be contiguous (they are written in place)")
    if pos.shape != (b,):
        raise ValueError("pos must be [B]")
    _hip.require_gpu(q, k_new, v_new, k_cache, v_cache, pos)
    q, k_new, v_new = q.contiguous(), k_new.contiguous(), v_new.contiguous()
    pos = pos.to(torch.int32).contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    max_len = k_cache.shape[2]
    out = torch.empty_like(q)
    lib = _hip.lib()
    ws_bytes = lib.ferrite_hip_decode_attention_workspace(b, h, max_len, d)
    ws = torch.empty(((ws_bytes + 3) // 4,), dtype=torch.float32, device=q.device) if ws_bytes > 0 else None
    rc = lib.ferrite_hip_decode_attention(
        q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), pos.data_ptr(),
        out.data_ptr(), b, h, max_len, d, _hip.dtype_code(q.dtype), float(scale), _hip.ptr(ws), max(ws_bytes, 0),
        _hip.stream_of(q),
    )
    _hip.check(rc, "ferrite_decode_attention")
    return out


def decode_attention_reference(q, k_new, v_new, k_cache, v_cache, pos, *, scale: float | None = None):
    """Torch restatement of engine.py:89-104: write the new rows at pos, then f32 scores over
    the whole cache masked to keys <= pos with -1e30, softmax, and P.V cast to q's dtype."""
    b, h, d = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    idx = torch.arange(b, device=q.device)
    p64 = pos.long()
    k_cache[idx, :, p64] = k_new.to(k_cache.dtype)
    v_cache[idx, :, p64] = v_new.to(v_cache.dtype)
    s = torch.einsum("bhd,bhkd->bhk", q.float(), k_cache.float()) * scale
    keys = torch.arange(k_cache.shape[2], device=q.device)[None, :]
    s = torch.where((keys <= p64[:, None])[:, None, :], s, torch.full_like(s, -1e30))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bhk,bhkd->bhd", p, v_cache.float()).to(q.dtype)
