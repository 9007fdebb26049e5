"""ferrite on MI355X: the causal flash attention, fused add+RMSNorm and blocked
matmul of ferrite.kernels, as hand-written gfx950 HIP kernels behind the same
Python API (reference: src/ferrite/__init__.py:7-13).

The kernels live in libferrite_hip.so (C ABI: include/ferrite_hip.h), built by
ferrite-tpu_amd/build_lib.py. Tensors are torch tensors on a ROCm device; torch
provides device memory and streams only.
"""

from ferrite import platform
from ferrite.kernels.flash_attention import flash_attention
from ferrite.kernels.matmul import matmul
from ferrite.kernels.rmsnorm import rmsnorm

__all__ = ["flash_attention", "matmul", "rmsnorm", "platform"]
__version__ = "0.1.0"
