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


def matmul_reference(x, y, *, out_dtype=None):
    """Torch baseline with the same numerics contract (f32 accumulation), matmul.py:129-131."""
    out = torch.matmul(x.float(), y.float())
    return out.to(to_torch_dtype(out_dtype) if out_dtype is not None else x.dtype)


def matmul_flops(m: int, n: int, k: int) -> int:
    return 2 * m * n * k
