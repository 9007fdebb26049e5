"""Blocked matmul with f32 accumulation on an MI355X MFMA kernel.

Reference: src/ferrite/kernels/matmul.py. Same public API, block-size
validation and custom VJP (dX = G Y^T, dY = X^T G through the same kernel,
matmul.py:89-107). The HIP kernel (csrc/matmul.hip: ferrite_hip_matmul) owns a
256x256 (bf16) or 128x128 (f32) output macro-tile per workgroup; ragged shapes
are zero-filled on load inside the kernel, which computes what the reference's
zero padding computes (matmul.py:59-63, :84-85) without copies.
"""

from __future__ import annotations

import torch

from ferrite import _hip, platform
from ferrite.kernels._compat import round_up, to_torch_dtype


def _pick_blocks(m: int, n: int, k: int, bm, bn, bk):
    """Block choice and ValueError of the reference (matmul.py:41-49); hints for the HIP kernel."""
    tile = platform.default_tile()
    big = 4 * tile
    bm = bm or (big if m >= big else round_up(m, platform.SUBLANES))
    bn = bn or (big if n >= big else round_up(n, platform.LANES))
    bk = bk or (big if k >= big else round_up(k, platform.LANES))
    if bm % platform.SUBLANES or bn % platform.LANES or bk % platform.LANES:
        raise ValueError(f"blocks must be multiples of ({platform.SUBLANES}, {platform.LANES}); got bm={bm} bn={bn} bk={bk}")
    return bm, bn, bk


def _transposed_ok(work, m: int, n: int, k: int, x_t: bool, tensors) -> bool:
    """Whether the DMA-fed kernel reads a transposed operand in place (ferrite_hip_matmul_ex's
    rule): bf16, K % 64 == 0, N % 8 == 0, M % 8 == 0 for a transposed x, 16-byte pointers."""
    return (work == torch.bfloat16 and k % 64 == 0 and n % 8 == 0 and (not x_t or m % 8 == 0)
            and all(t.data_ptr() % 16 == 0 for t in tensors))


def _mm(xs, ys, m: int, n: int, k: int, x_t: bool, y_t: bool, out_dtype):
    """out[m, n] = op(xs) @ op(ys) on the HIP kernel. xs holds x [m, k], or its transpose [k, m]
    when x_t; ys holds y [k, n], or [n, k] when y_t. A transposed operand the kernel cannot read
    in place is transposed into a copy first."""
    work = torch.promote_types(xs.dtype, ys.dtype)
    xs = xs.to(work).contiguous()
    ys = ys.to(work).contiguous()
    kernel_out = out_dtype if out_dtype in (torch.float32, torch.bfloat16) else torch.float32
    out = torch.empty((m, n), dtype=kernel_out, device=xs.device)
    if (x_t or y_t) and not _transposed_ok(work, m, n, k, x_t, (xs, ys, out)):
        if x_t:
            xs, x_t = xs.t().contiguous(), False
        if y_t:
            ys, y_t = ys.t().contiguous(), False
    if m and n:
        if k == 0:
            out.zero_()
        else:
            lib = _hip.lib()
            code = _hip.dtype_code(work)
            ws_bytes = lib.ferrite_hip_matmul_workspace(m, n, k, code)
            ws = torch.empty(((ws_bytes + 3) // 4,), dtype=torch.float32, device=xs.device) if ws_bytes > 0 else None
            rc = lib.ferrite_hip_matmul_ex(
                xs.data_ptr(), ys.data_ptr(), out.data_ptr(), m, n, k, int(x_t), int(y_t), code,
                _hip.dtype_code(kernel_out), _hip.ptr(ws), max(ws_bytes, 0), _hip.stream_of(xs),
            )
            _hip.check(rc, "ferrite_matmul")
    return out if kernel_out == out_dtype else out.to(out_dtype)


def _matmul_impl(x, y, block_m=None, block_n=None, block_k=None, out_dtype=None):
    if x.ndim != 2 or y.ndim != 2 or x.shape[1] != y.shape[0]:
        raise ValueError(f"expected [M,K] @ [K,N], got {tuple(x.shape)} @ {tuple(y.shape)}")
    m, k = x.shape
    _, n = y.shape
    out_dtype = to_torch_dtype(out_dtype) if out_dtype is not None else x.dtype
    _pick_blocks(m, n, k, block_m, block_n, block_k)
    _hip.require_gpu(x, y)
    # Mixed operand dtypes are promoted as jnp.dot would; widening bf16 to f32 is exact.
    return _mm(x, y, m, n, k, False, False, out_dtype)


class _MatmulFn(torch.autograd.Function):
    """`_matmul_vjp` of the reference (matmul.py:89-107): non-differentiable cfg. The two
    backward products read y and x transposed in place (no materialised transposes)."""

    @staticmethod
    def forward(ctx, x, y, cfg):
        bm, bn, bk, out_dtype = cfg
        ctx.save_for_backward(x, y)
        return _matmul_impl(x, y, bm, bn, bk, out_dtype)

    @staticmethod
    def backward(ctx, g):
        x, y = ctx.saved_tensors
        m, k = x.shape
        n = y.shape[1]
        dx = _mm(g.to(x.dtype), y, m, k, n, False, True, x.dtype)  # g [m,n] @ y^T (y stored [k,n])
        dy = _mm(x, g.to(y.dtype), k, n, m, True, False, y.dtype)  # x^T (x stored [m,k]) @ g [m,n]
        return dx, dy, None


def matmul(x, y, *, block_m: int | None = None, block_n: int | None = None, block_k: int | None = None, out_dtype=None):
    """``x @ y`` for 2-D ``x: [M, K]`` and ``y: [K, N]`` with f32 accumulation (matmul.py:110-126).

    Any shape is accepted; ragged edges behave as zero padding. Differentiable.
    """
    cfg = (block_m, block_n, block_k, out_dtype)
    return _MatmulFn.apply(x, y, cfg)


def _mm_gelu(xs, ys, aux, m: int, n: int, k: int, x_t: bool, y_t: bool, mode: int):
    """bf16 [m, n] product of op(xs) @ op(ys) with a GELU epilogue (ferrite_hip_matmul_gelu):
    mode GELU writes the pre-activation into aux and returns gelu of it; mode GELU_GRAD
    returns the product times gelu'(aux)."""
    xs, ys = xs.contiguous(), ys.contiguous()
    out = torch.empty((m, n), dtype=torch.bfloat16, device=xs.device)
    if (x_t or y_t) and not _transposed_ok(torch.bfloat16, m, n, k, x_t, (xs, ys, out)):
        if x_t:
            xs, x_t = xs.t().contiguous(), False
        if y_t:
            ys, y_t = ys.t().contiguous(), False
    lib = _hip.lib()
    ws_bytes = lib.ferrite_hip_matmul_workspace(m, n, k, _hip.BF16)
    ws = torch.empty(((ws_bytes + 3) // 4,), dtype=torch.float32, device=xs.device) if ws_bytes > 0 else None
    rc = lib.ferrite_hip_matmul_gelu(xs.data_ptr(), ys.data_ptr(), out.data_ptr(), aux.data_ptr(), m, n, k, int(x_t),
                                     int(y_t), mode, _hip.ptr(ws), max(ws_bytes, 0), _hip.stream_of(xs))
    _hip.check(rc, "ferrite_matmul_gelu")
    return out


class _GeluMlpFn(torch.autograd.Function):
    """gelu(x @ w1) @ w2 with the GELU in the matmul epilogues. Forward: the up-projection
    stores u = x @ w1 and a = gelu(u) in one pass. Backward: the product g @ w2^T is scaled by
    gelu'(u) as it is stored, so neither direction runs an elementwise GELU pass. The other
    products are the matmul VJP's (transposed operands read in place)."""

    @staticmethod
    def forward(ctx, x, w1, w2):
        t, d = x.shape
        f, e = w1.shape[1], w2.shape[1]
        u = torch.empty((t, f), dtype=torch.bfloat16, device=x.device)
        a = _mm_gelu(x, w1, u, t, f, d, False, False, _hip.GELU)
        out = _mm(a, w2, t, e, f, False, False, torch.bfloat16)
        ctx.save_for_backward(x, w1, w2, u, a)
        return out

    @staticmethod
    def backward(ctx, g):
        x, w1, w2, u, a = ctx.saved_tensors
        t, d = x.shape
        f, e = w1.shape[1], w2.shape[1]
        g = g.to(torch.bfloat16).contiguous()
        du = _mm_gelu(g, w2, u, t, f, e, False, True, _hip.GELU_GRAD)  # (g @ w2^T) * gelu'(u)
        dw2 = _mm(a, g, f, e, t, True, False, torch.bfloat16)  # a^T @ g
        dx = _mm(du, w1, t, d, f, False, True, torch.bfloat16)  # du @ w1^T
        dw1 = _mm(x, du, d, f, t, True, False, torch.bfloat16)  # x^T @ du
        return dx, dw1, dw2


def mlp_gelu(x, w1, w2):
    """``gelu(x @ w1) @ w2`` (the tanh GELU, jax.nn.gelu(approximate=True)) for bf16
    ``x: [..., d]``, ``w1: [d, f]``, ``w2: [f, e]``, differentiable. The transformer MLP of
    model/gpt.py:141, with the GELU and its derivative applied inside the matmul kernels."""
    if x.dtype != torch.bfloat16 or w1.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16:
        raise ValueError("mlp_gelu takes bf16 x, w1, w2")
    if w1.ndim != 2 or w2.ndim != 2 or x.shape[-1] != w1.shape[0] or w1.shape[1] != w2.shape[0]:
        raise ValueError(f"expected [..., d] @ [d, f] @ [f, e]; got {tuple(x.shape)}, {tuple(w1.shape)}, {tuple(w2.shape)}")
    _hip.require_gpu(x, w1, w2)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[0] == 0:
        return x.new_zeros((*lead, w2.shape[1]))
    return _GeluMlpFn.apply(x2, w1, w2).reshape(*lead, w2.shape[1])


def matmul_reference(x, y, *, out_dtype=None):
    """Torch baseline with the same numerics contract (f32 accumulation), matmul.py:129-131."""
    out = torch.matmul(x.float(), y.float())
    return out.to(to_torch_dtype(out_dtype) if out_dtype is not None else x.dtype)


def matmul_flops(m: int, n: int, k: int) -> int:
    return 2 * m * n * k
