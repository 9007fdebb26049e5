"""Causal flash attention, forward and backward, on MI355X HIP kernels.

Reference: src/ferrite/kernels/flash_attention.py. Same public names, arguments,
defaults and ValueError conditions; the custom VJP wiring of the reference
(`_flash` with non-differentiable (causal, scale, block_sizes), residuals
(q, k, v, out, lse), backward = delta + dK/dV kernel + dQ kernel,
flash_attention.py:315-333) is a torch.autograd.Function here.

Kernels (csrc/attention.hip, through include/ferrite_hip.h):
  forward   ferrite_hip_attn_fwd_ex       -> O [B,H,S,D], lse f32 [B,H,S]
  delta     ferrite_hip_attn_bwd_delta    -> rowsum(f32 dO * f32 O)
  dK, dV    ferrite_hip_attn_bwd_dkv_ex
  dQ        ferrite_hip_attn_bwd_dq_ex (or _dq_delta_ex, computing delta)
The _ex entry points take a workspace (sized by ferrite_hip_attn_fwd_workspace /
_bwd_workspace, zero bytes where it is not used) in which the long-context kernels
split their longest tiles between the two workgroups of a CU.
lse and delta are compact [B,H,S] f32 rather than the reference's
lane-replicated [B,H,S,128] (flash_attention.py:156-160, :329).

Block sizes are validated exactly as in the reference and otherwise treated as
hints: the HIP kernels use their own tiles (128-row query tiles in 32-row MFMA
wave tiles), which changes only the f32 summation order.
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np
import torch

from ferrite import _hip, platform

NUM_LANES = platform.LANES
# Large negative finite value the reference uses for masked scores (flash_attention.py:43-44).
MASK_VALUE = -0.7 * float(np.finfo(np.float32).max)


@dataclasses.dataclass(frozen=True)
class BlockSizes:
    """Tile sizes. ``block_q`` is a multiple of 8, ``block_k`` a multiple of 128 (flash_attention.py:49-62)."""

    block_q: int = 128
    block_k: int = 128
    block_q_bwd: int = 128
    block_k_bwd: int = 128

    @classmethod
    def for_device(cls) -> "BlockSizes":
        t = platform.default_tile()
        return cls(t, t, t, t)


def _on_or_below_diag(qi: int, bq: int, ki: int, bk: int) -> bool:
    """True when block (qi, ki) has at least one unmasked (col <= row) entry (flash_attention.py:65-67)."""
    return (qi + 1) * bq - 1 >= ki * bk


# --------------------------------------------------------------------------
# kernel launches
# --------------------------------------------------------------------------


# Workspaces of the long-context split kernels (partial states and per-pair counts), one per
# (pass, device, stream, size), zero-filled once: the kernels leave the counts even, as they found
# them. The forward ("fwd") and the backward's dQ and dK/dV ("bwd", which take turns with one
# buffer) keep separate ones. A workspace first needed inside a graph capture is allocated there
# (its zero fill is then part of the graph) and not kept.
_WORKSPACES: dict[tuple, torch.Tensor] = {}


def _workspace(kind: str, nbytes: int, device: torch.device) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    stream = torch.cuda.current_stream(device)
    key = (kind, device, stream.cuda_stream, nbytes)
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        if not torch.cuda.is_current_stream_capturing():
            _WORKSPACES[key] = ws
    return ws


def _ws_args(ws: torch.Tensor | None) -> tuple:
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel())


def _flash_forward(q, k, v, *, causal: bool, scale: float, bs: BlockSizes | None = None):
    """O and the compact logsumexp. Reference: _flash_forward, flash_attention.py:130-175."""
    _hip.require_gpu(q, k, v)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    b, h, sq, d = q.shape
    sk = k.shape[2]
    out = torch.empty_like(q)
    lse = torch.empty((b, h, sq), dtype=torch.float32, device=q.device)
    lib, dt = _hip.lib(), _hip.dtype_code(q.dtype)
    ws = _workspace("fwd", lib.ferrite_hip_attn_fwd_workspace(b, h, sq, sk, d, dt, int(causal)), q.device)
    rc = lib.ferrite_hip_attn_fwd_ex(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
        b, h, sq, sk, d, dt, int(causal), float(scale), *_ws_args(ws), _hip.stream_of(q),
    )
    _hip.check(rc, "ferrite_flash_attention_fwd")
    return out, lse


def _flash_delta(out, do):
    """delta = rowsum(f32 dO * f32 O), flash_attention.py:328."""
    out, do = out.contiguous(), do.contiguous()
    b, h, s, d = out.shape
    delta = torch.empty((b, h, s), dtype=torch.float32, device=out.device)
    rc = _hip.lib().ferrite_hip_attn_bwd_delta(
        out.data_ptr(), do.data_ptr(), delta.data_ptr(), b, h, s, d, _hip.dtype_code(out.dtype), _hip.stream_of(out)
    )
    _hip.check(rc, "ferrite_flash_attention_bwd_delta")
    return delta


def _flash_backward_fused(q, k, v, out, do, lse, *, causal: bool, scale: float):
    """dQ, dK, dV with delta (flash_attention.py:328-329) computed inside the dQ kernel from O
    and dO and handed to dK/dV, which therefore runs second: no separate delta pass."""
    _hip.require_gpu(q, k, v, out, do, lse)
    q, k, v, out, do, lse = (t.contiguous() for t in (q, k, v, out, do, lse))
    b, h, sq, d = q.shape
    sk = k.shape[2]
    dt = _hip.dtype_code(q.dtype)
    stream = _hip.stream_of(q)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    delta = torch.empty((b, h, sq), dtype=torch.float32, device=q.device)
    lib = _hip.lib()
    wsa = _ws_args(_workspace("bwd", lib.ferrite_hip_attn_bwd_workspace(b, h, sq, sk, d, dt, int(causal)), q.device))
    rc = lib.ferrite_hip_attn_bwd_dq_delta_ex(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), do.data_ptr(), lse.data_ptr(), delta.data_ptr(),
        dq.data_ptr(), b, h, sq, sk, d, dt, int(causal), float(scale), *wsa, stream,
    )
    _hip.check(rc, "ferrite_flash_attention_bwd_dq")
    rc = lib.ferrite_hip_attn_bwd_dkv_ex(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), lse.data_ptr(), delta.data_ptr(),
        dk.data_ptr(), dv.data_ptr(), b, h, sq, sk, d, dt, int(causal), float(scale), *wsa, stream,
    )
    _hip.check(rc, "ferrite_flash_attention_bwd_dkv")
    return dq, dk, dv


def _flash_backward(q, k, v, do, lse, delta, *, causal: bool, scale: float, bs: BlockSizes | None = None):
    """dQ, dK, dV. Reference: _flash_backward, flash_attention.py:246-307 (two kernels, no atomics)."""
    _hip.require_gpu(q, k, v, do, lse, delta)
    q, k, v, do = q.contiguous(), k.contiguous(), v.contiguous(), do.contiguous()
    lse, delta = lse.contiguous(), delta.contiguous()
    b, h, sq, d = q.shape
    sk = k.shape[2]
    dt = _hip.dtype_code(q.dtype)
    stream = _hip.stream_of(q)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    lib = _hip.lib()
    wsa = _ws_args(_workspace("bwd", lib.ferrite_hip_attn_bwd_workspace(b, h, sq, sk, d, dt, int(causal)), q.device))
    rc = lib.ferrite_hip_attn_bwd_dkv_ex(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), lse.data_ptr(), delta.data_ptr(),
        dk.data_ptr(), dv.data_ptr(), b, h, sq, sk, d, dt, int(causal), float(scale), *wsa, stream,
    )
    _hip.check(rc, "ferrite_flash_attention_bwd_dkv")
    rc = lib.ferrite_hip_attn_bwd_dq_ex(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), lse.data_ptr(), delta.data_ptr(),
        dq.data_ptr(), b, h, sq, sk, d, dt, int(causal), float(scale), *wsa, stream,
    )
    _hip.check(rc, "ferrite_flash_attention_bwd_dq")
    return dq, dk, dv


# --------------------------------------------------------------------------
# custom VJP and public API
# --------------------------------------------------------------------------


class _Flash(torch.autograd.Function):
    """`_flash` of the reference (flash_attention.py:315-333): non-differentiable (causal, scale, bs)."""

    @staticmethod
    def forward(ctx, q, k, v, causal: bool, scale: float, bs: BlockSizes):
        # The kernels read dense [B, H, S, D]; the dense copies are what the backward re-reads.
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        out, lse = _flash_forward(q, k, v, causal=causal, scale=scale, bs=bs)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.causal, ctx.scale, ctx.bs = causal, scale, bs
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, out, lse = ctx.saved_tensors
        do = do.to(out.dtype).contiguous()
        dq, dk, dv = _flash_backward_fused(q, k, v, out, do, lse, causal=ctx.causal, scale=ctx.scale)
        return dq, dk, dv, None, None, None


def _validate(q, k, v, causal, bs):
    """ValueErrors of the reference (flash_attention.py:336-353), same conditions and order."""
    if not (q.ndim == 4 and k.shape == v.shape and q.shape[:2] == k.shape[:2] and q.shape[3] == k.shape[3]):
        raise ValueError(f"expected q,k,v as [b,h,s,d] with matching b,h,d; got {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, v must share a dtype")
    d = q.shape[3]
    if d % NUM_LANES and d > NUM_LANES:
        raise ValueError(f"head_dim must be <= {NUM_LANES} or a multiple of it; got {d}")
    if causal and q.shape[2] != k.shape[2]:
        raise ValueError("causal attention needs equal q and k sequence lengths")
    for name, blk, dim, mult in [
        ("block_q", bs.block_q, q.shape[2], platform.SUBLANES),
        ("block_k", bs.block_k, k.shape[2], NUM_LANES),
        ("block_q_bwd", bs.block_q_bwd, q.shape[2], platform.SUBLANES),
        ("block_k_bwd", bs.block_k_bwd, k.shape[2], NUM_LANES),
    ]:
        if blk % mult or dim % blk:
            raise ValueError(f"{name}={blk} must be a multiple of {mult} and divide the sequence length {dim}")


def flash_attention(q, k, v, *, causal: bool = True, scale: float | None = None, block_sizes: BlockSizes | None = None):
    """Memory-efficient attention ``softmax(q k^T * scale) v`` with exact numerics.

    Differentiable through autograd (custom backward with HIP dK/dV and dQ
    kernels). Shapes ``[batch, heads, seq, head_dim]``; sequence lengths must be
    multiples of the block sizes, as in the reference (flash_attention.py:356-367).
    """
    bs = block_sizes or BlockSizes()
    _validate(q, k, v, causal, bs)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return _Flash.apply(q, k, v, bool(causal), float(scale), bs)


class _FlashQKV(torch.autograd.Function):
    """Causal attention on the token-major projection [B, S, 3, H, D] -> [B, S, H, D], the
    head transposes of model/gpt.py:137-138 folded into the kernels' addressing."""

    @staticmethod
    def forward(ctx, qkv, heads, scale):
        b, s, three, h, d = qkv.shape
        o = torch.empty((b, s, h, d), dtype=qkv.dtype, device=qkv.device)
        lse = torch.empty((b, h, s), dtype=torch.float32, device=qkv.device)
        rc = _hip.lib().ferrite_hip_attn_fwd_qkv(qkv.data_ptr(), o.data_ptr(), lse.data_ptr(), b, s, h, d,
                                                 float(scale), _hip.stream_of(qkv))
        _hip.check(rc, "ferrite_flash_attention_fwd")
        ctx.save_for_backward(qkv, o, lse)
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx, do):
        qkv, o, lse = ctx.saved_tensors
        b, s, _, h, d = qkv.shape
        do = do.to(o.dtype).contiguous()
        dqkv = torch.empty_like(qkv)
        delta = torch.empty((b, h, s), dtype=torch.float32, device=qkv.device)
        rc = _hip.lib().ferrite_hip_attn_bwd_qkv(qkv.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(),
                                                 delta.data_ptr(), dqkv.data_ptr(), b, s, h, d, float(ctx.scale),
                                                 _hip.stream_of(qkv))
        _hip.check(rc, "ferrite_flash_attention_bwd")
        return dqkv, None, None


def flash_attention_qkv_supported(qkv, heads: int) -> bool:
    """Whether flash_attention_qkv takes this projection: bf16 on the GPU, head_dim 64 or 128,
    sequence length a multiple of 64."""
    if qkv.ndim != 3 or qkv.shape[-1] % (3 * heads):
        return False
    d = qkv.shape[-1] // (3 * heads)
    return qkv.dtype == torch.bfloat16 and qkv.is_cuda and d in (64, 128) and qkv.shape[1] % 64 == 0


def flash_attention_qkv(qkv, heads: int, *, scale: float | None = None):
    """Causal ``softmax(q k^T * scale) v`` for the fused projection ``qkv: [B, S, 3 * H * D]``
    (columns ordered (q|k|v, head, dim), as model/gpt.py:136-137 splits them), returning
    ``[B, S, H * D]`` in the token-major order the output projection reads (gpt.py:138).
    Differentiable; the same kernels and numbers as flash_attention on transposed copies,
    without the copies. bf16, head_dim 64 or 128, sequence length a multiple of 64."""
    if not flash_attention_qkv_supported(qkv, heads):
        raise ValueError(f"flash_attention_qkv needs bf16 [B, S, 3*H*D] on the GPU with D in (64, 128) and S % 64 == 0; "
                         f"got {tuple(qkv.shape)} {qkv.dtype} for {heads} heads")
    b, s, c = qkv.shape
    d = c // (3 * heads)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    o = _FlashQKV.apply(qkv.contiguous().view(b, s, 3, heads, d), heads, float(scale))
    return o.view(b, s, heads * d)


def flash_attention_reference(q, k, v, *, causal: bool = True, scale: float | None = None):
    """Materialised-scores attention in f32 with torch ops (the reference's XLA route,
    flash_attention.py:370-380). Not used by the HIP path."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    qf, kf, vf = q.float(), k.float(), v.float()
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale
    if causal:
        sq, sk = q.shape[2], k.shape[2]
        mask = torch.ones((sq, sk), dtype=torch.bool, device=q.device).tril(diagonal=sk - sq)
        s = torch.where(mask, s, torch.full_like(s, MASK_VALUE))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vf).to(q.dtype)


def attention_flops(b: int, h: int, sq: int, sk: int, d: int, *, causal: bool, backward: bool = False) -> int:
    """FLOPs for one forward (and optionally backward) pass, skipped blocks free (flash_attention.py:383-390)."""
    frac = 0.5 if causal else 1.0
    fwd = 4 * b * h * sq * sk * d * frac
    if not backward:
        return int(fwd)
    return int(fwd * 2.5)
