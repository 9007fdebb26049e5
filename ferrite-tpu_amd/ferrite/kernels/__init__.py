"""Public kernel API (reference: src/ferrite/kernels/__init__.py:1-12)."""

from ferrite.kernels.flash_attention import BlockSizes, attention_flops, flash_attention, flash_attention_reference
from ferrite.kernels.matmul import matmul, matmul_flops, matmul_reference
from ferrite.kernels.rmsnorm import rmsnorm, rmsnorm_reference

__all__ = [
    "BlockSizes",
    "attention_flops",
    "flash_attention",
    "flash_attention_reference",
    "matmul",
    "matmul_flops",
    "matmul_reference",
    "rmsnorm",
    "rmsnorm_reference",
]
