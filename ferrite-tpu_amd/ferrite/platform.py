"""Platform constants and MI355X roofline peaks.

Reference: src/ferrite/platform.py. The tiling constants keep the reference's
values (LANES = 128, SUBLANES = 8, default_tile() = 128) because the public API
validates block sizes against them (flash_attention.py:336-353, matmul.py:41-49);
on MI355X block sizes are hints and the HIP kernels choose their own tiles.
The peaks describe one MI355X (gfx950): AMD's published dense figures.
"""

from __future__ import annotations

import contextlib
import dataclasses
import os
from typing import Iterator

import torch

LANES = 128  # block-size validation unit of the reference API (last block dim)
SUBLANES = 8  # second-to-last block dim unit of the reference API


def backend() -> str:
    """'rocm' when a ROCm GPU is visible to torch, else 'cpu'."""
    if torch.version.hip is not None and torch.cuda.is_available():
        return "rocm"
    return "cpu"


def is_tpu() -> bool:
    return False


def is_rocm() -> bool:
    return backend() == "rocm"


def device_kind() -> str:
    if is_rocm():
        return torch.cuda.get_device_name(0)
    return "cpu"


def num_devices() -> int:
    return torch.cuda.device_count() if is_rocm() else 0


def mxu_width() -> int:
    """Width used by the reference for default tiles; kept at 128 so BlockSizes.for_device() matches."""
    return 128


def default_tile() -> int:
    return max(LANES, mxu_width())


@dataclasses.dataclass(frozen=True)
class Peaks:
    """Per-device peak numbers for the roofline."""

    name: str
    bf16_flops: float  # dense MFMA FLOP/s
    fp32_flops: float  # dense fp32 MFMA FLOP/s
    hbm_bytes_per_s: float
    hbm_bytes: float
    lds_bytes: float  # per CU
    cores: int  # compute units

    @property
    def ridge_point(self) -> float:
        """Arithmetic intensity (FLOP/byte) at which bf16 compute and HBM limits meet."""
        return self.bf16_flops / self.hbm_bytes_per_s


MI355X = Peaks(
    name="MI355X",
    bf16_flops=2.5166e15,
    fp32_flops=157.3e12,
    hbm_bytes_per_s=8.0e12,
    hbm_bytes=288e9,
    lds_bytes=160 * 1024,
    cores=256,
)

_CHIPS = {"MI355X": MI355X, "GFX950": MI355X}


def peaks(chip: str | None = None) -> Peaks | None:
    """Roofline peaks for `chip` (e.g. 'MI355X'), or for the attached GPU (None off-GPU)."""
    if chip is not None:
        return _CHIPS[chip.upper()]
    if not is_rocm():
        return None
    arch = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")
    return MI355X if arch.startswith("gfx950") else None


@contextlib.contextmanager
def interpret_mode(force: bool | None = None) -> Iterator[bool]:
    """The reference's TPU interpret-mode switch (platform.py:111-123). MI355X has no
    kernel interpreter, so this is a no-op that yields False; it exists so callers
    written against the reference keep working."""
    yield False


def describe() -> dict:
    """Small dict describing the platform; written into every results file."""
    out = {
        "backend": backend(),
        "device_kind": device_kind(),
        "num_devices": num_devices(),
        "torch_version": torch.__version__,
        "hip_version": torch.version.hip,
        "host_cores": len(os.sched_getaffinity(0)),
    }
    p = peaks()
    if p is not None:
        out.update(
            chip=p.name,
            compute_units=p.cores,
            peak_bf16_tflops=p.bf16_flops / 1e12,
            peak_fp32_tflops=p.fp32_flops / 1e12,
            peak_hbm_gbps=p.hbm_bytes_per_s / 1e9,
            lds_kib_per_cu=p.lds_bytes / 1024,
            ridge_point_flop_per_byte=p.ridge_point,
        )
    return out
