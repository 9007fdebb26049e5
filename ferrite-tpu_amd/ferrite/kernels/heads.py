"""Token-major <-> head-major layout changes around attention, on HIP kernels.

Reference: the transposes of src/ferrite/model/gpt.py:137-138 (qkv split into
[B, H, S, hd] heads, attention output back to [B, S, d]), which XLA lowers to
copy fusions. csrc/layout.hip moves 16-byte vectors with both sides
coalesced; each direction is the other's backward.
"""

from __future__ import annotations

import ctypes

import torch

from ferrite import _hip


def _ptr_array(tensors):
    arr = (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])
    return ctypes.cast(arr, ctypes.c_void_p), arr


def _split(x, groups: int, heads: int):
    b, s, w = x.shape
    d = w // (groups * heads)
    x = x.contiguous()
    outs = [torch.empty((b, heads, s, d), dtype=x.dtype, device=x.device) for _ in range(groups)]
    p, _keep = _ptr_array(outs)
    rc = _hip.lib().ferrite_hip_heads_split(x.data_ptr(), p, b, s, groups, heads, d, _hip.dtype_code(x.dtype),
                                            _hip.stream_of(x))
    _hip.check(rc, "ferrite_heads_split")
    return outs


def _merge(parts):
    parts = [t.contiguous() for t in parts]
    b, h, s, d = parts[0].shape
    out = torch.empty((b, s, len(parts) * h * d), dtype=parts[0].dtype, device=parts[0].device)
    p, _keep = _ptr_array(parts)
    rc = _hip.lib().ferrite_hip_heads_merge(p, out.data_ptr(), b, s, len(parts), h, d, _hip.dtype_code(out.dtype),
                                            _hip.stream_of(out))
    _hip.check(rc, "ferrite_heads_merge")
    return out


class _SplitHeads(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, groups, heads):
        return tuple(_split(x, groups, heads))

    @staticmethod
    def backward(ctx, *grads):
        grads = [g if g is not None else None for g in grads]
        if any(g is None for g in grads):
            ref = next(g for g in grads if g is not None)
            grads = [torch.zeros_like(ref) if g is None else g for g in grads]
        return _merge(grads), None, None


class _MergeHeads(torch.autograd.Function):
    @staticmethod
    def forward(ctx, *parts):
        ctx.groups, ctx.heads = len(parts), parts[0].shape[1]
        return _merge(parts)

    @staticmethod
    def backward(ctx, g):
        return tuple(_split(g, ctx.groups, ctx.heads))


def split_heads(x: torch.Tensor, groups: int, heads: int):
    """[B, S, groups*heads*D] -> `groups` contiguous tensors [B, heads, S, D] (differentiable)."""
    if x.ndim != 3 or x.shape[2] % (groups * heads):
        raise ValueError(f"expected [B, S, groups*heads*D]; got {tuple(x.shape)} for groups={groups}, heads={heads}")
    if not 1 <= groups <= 4:
        raise ValueError("groups must be 1..4")
    _hip.require_gpu(x)
    return _SplitHeads.apply(x, groups, heads)


def merge_heads(*parts: torch.Tensor) -> torch.Tensor:
    """Tensors [B, H, S, D] -> [B, S, len(parts)*H*D] (differentiable)."""
    if not 1 <= len(parts) <= 4 or any(p.shape != parts[0].shape or p.ndim != 4 for p in parts):
        raise ValueError("merge_heads takes 1..4 tensors of one [B, H, S, D] shape")
    _hip.require_gpu(*parts)
    return _MergeHeads.apply(*parts)
