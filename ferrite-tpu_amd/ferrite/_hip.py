"""ctypes binding of libferrite_hip.so, the C ABI declared in include/ferrite_hip.h.

This is the only place Python touches the native library. Tensors cross as raw
device pointers plus sizes; the stream is torch's current HIP stream on the
tensors' device, so the kernels order correctly with surrounding torch work.
There is no fallback: if the library is missing or a tensor is not on a ROCm
GPU, the call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libferrite_hip.so")

F32 = 0
BF16 = 1
RMSNORM_BWD_SCRATCH_BYTES = 8 << 20  # FERRITE_RMSNORM_BWD_SCRATCH_BYTES
GELU = 1
GELU_GRAD = 2
OK = 0

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_f32 = ctypes.c_float
_vp = ctypes.c_void_p

# name -> (restype, argtypes); must match include/ferrite_hip.h.
SIGNATURES: dict[str, tuple] = {
    "ferrite_hip_last_error": (ctypes.c_char_p, []),
    "ferrite_hip_version": (ctypes.c_char_p, []),
    "ferrite_hip_add_rmsnorm": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp]),
    "ferrite_hip_rmsnorm": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp]),
    "ferrite_hip_rmsnorm_bwd_workspace": (_c_i64, [_c_i64, _c_i64]),
    "ferrite_hip_rmsnorm_bwd": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_f32, _vp],
    ),
    "ferrite_hip_rmsnorm_bwd_noalloc": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_f32, _vp],
    ),
    "ferrite_hip_stream_copy2": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _vp]),
    "ferrite_hip_stream_read": (_c_int, [_vp, _c_i64, _vp, _c_int, _vp]),
    "ferrite_hip_stream_fill": (_c_int, [_vp, _c_i64, ctypes.c_uint32, _c_int, _vp]),
    "ferrite_hip_mfma_ceiling": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp]),
    "ferrite_hip_matmul": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _vp]),
    "ferrite_hip_matmul_workspace": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_int]),
    "ferrite_hip_matmul_ex": (
        _c_int,
        [_vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _c_i64, _vp],
    ),
    "ferrite_hip_decode_attention_workspace": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "ferrite_hip_decode_attention": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_f32, _vp, _c_i64, _vp],
    ),
    "ferrite_hip_heads_split": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _vp]),
    "ferrite_hip_heads_merge": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _vp]),
    "ferrite_hip_cross_entropy_fwd": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _vp]),
    "ferrite_hip_cross_entropy_bwd": (_c_int, [_vp, _vp, _vp, _vp, _c_f32, _vp, _c_i64, _c_i64, _c_int, _vp]),
    "ferrite_hip_adamw_workspace": (_c_i64, [_c_i64]),
    "ferrite_hip_adamw": (
        _c_int,
        [_c_i64, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32,
         _c_i64, _vp, _vp, _vp, _vp],
    ),
    "ferrite_hip_attn_fwd": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp],
    ),
    "ferrite_hip_attn_fwd_workspace": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "ferrite_hip_attn_fwd_ex": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp, _c_i64, _vp],
    ),
    "ferrite_hip_attn_bwd_delta": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _vp]),
    "ferrite_hip_attn_bwd_workspace": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "ferrite_hip_attn_bwd_dkv_ex": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp,
         _c_i64, _vp],
    ),
    "ferrite_hip_attn_bwd_dq_ex": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp, _c_i64,
         _vp],
    ),
    "ferrite_hip_attn_bwd_dq_delta_ex": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp,
         _c_i64, _vp],
    ),
    "ferrite_hip_attn_bwd_dkv": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp],
    ),
    "ferrite_hip_attn_bwd_dq": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp],
    ),
    "ferrite_hip_matmul_gelu": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _vp, _c_i64, _vp],
    ),
    "ferrite_hip_attn_fwd_qkv": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32, _vp]),
    "ferrite_hip_attn_bwd_qkv": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32, _vp],
    ),
    "ferrite_hip_attn_bwd_dq_delta": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f32, _vp],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python ferrite-tpu_amd/build_lib.py` "
                    "(or __graft_entry__.build()). ferrite has no non-HIP fallback."
                )
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def last_error() -> str:
    return lib().ferrite_hip_last_error().decode()


def check(rc: int, what: str) -> None:
    if rc != OK:
        raise RuntimeError(f"{what} failed (code {rc}): {last_error()}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return BF16
    if dtype == torch.float32:
        return F32
    raise ValueError(f"ferrite's HIP kernels take float32 or bfloat16 tensors; got {dtype}")


def require_gpu(*tensors: torch.Tensor) -> None:
    dev = None
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                f"ferrite's HIP kernels run on a ROCm GPU; got a tensor on {t.device}. "
                "There is no CPU path (use the *_reference functions for CPU math)."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
