"""Per-kernel roofline on MI355X: which pipe bounds a launch, and how close it runs to that pipe.

A launch does ``flops`` of matrix work in one precision and must move ``bytes`` through HBM
(both algorithmic: the work and the bytes the operation itself needs, counted the way the
kernels' callers count them, causal-skipped tiles free). At the part's peaks the matrix cores
need ``flops / peak[precision]`` seconds and HBM needs ``bytes / hbm_peak`` seconds. The
larger of the two is the floor on the launch's time, and it names the bound ("mfma" or
"hbm"). ``frac`` is that floor over the measured time, i.e. the achieved rate in the bound's
unit over the bound's peak, the figure bench.py reports as ``roofline.frac``.

Measured HBM traffic comes from rocprofv3's ``FETCH_SIZE`` and ``WRITE_SIZE`` counters (KiB per
dispatch). On gfx950 each counter reads a fixed multiple of the bytes really moved, found by
profiling a plain device copy of known size: :func:`traffic_bytes` applies those factors.
Traffic above the algorithmic bytes means re-reads (or spills), which the report shows as
``traffic / bytes``.

Peaks: the MI355X's published dense figures (no 2:1 sparsity), per MFMA input precision.
Interface names follow the reference's ferrite.profiling (src/ferrite/profiling/roofline.py:
``analyze``, ``format_table``, a point type), so callers written against it keep working.
"""

from __future__ import annotations

import dataclasses

from ferrite import platform

# Dense matrix-core peaks of one MI355X, FLOP/s (OP/s for int8), by input precision.
MI355X_MFMA_PEAKS = {
    "bf16": 2.5166e15,
    "fp16": 2.5166e15,
    "fp8": 5.0332e15,
    "fp6": 10.1e15,
    "fp4": 10.1e15,
    "int8": 5.0332e15,
    "fp32": 157.3e12,
    "fp64": 78.6e12,
}


def traffic_bytes(fetch_kib: float, write_kib: float, fetch_scale: float = 2.0, write_scale: float = 1.0) -> float:
    """HBM bytes of one dispatch from rocprofv3 ``FETCH_SIZE`` / ``WRITE_SIZE`` readings (KiB).

    The default scales are this part's calibration: a 256 MiB device copy reads FETCH_SIZE
    131,085 KiB and WRITE_SIZE 262,144 KiB per dispatch for 262,144 KiB moved each way."""
    return (fetch_kib * fetch_scale + write_kib * write_scale) * 1024.0


@dataclasses.dataclass(frozen=True)
class KernelRoofline:
    """One kernel launch against the roofline of one device (or ``devices`` of them)."""

    name: str
    flops: float
    bytes: float
    seconds: float
    precision: str = "bf16"
    traffic: float | None = None  # measured HBM bytes per launch (rocprofv3), if known
    mfma_peak: float | None = None  # FLOP/s of the matrix cores at `precision`
    hbm_peak: float | None = None  # bytes/s

    @property
    def mfma_floor_s(self) -> float | None:
        return None if not self.mfma_peak else self.flops / self.mfma_peak

    @property
    def hbm_floor_s(self) -> float | None:
        return None if not self.hbm_peak else self.bytes / self.hbm_peak

    @property
    def bound(self) -> str:
        """'mfma' or 'hbm': the pipe whose floor is longer; 'unknown' without peaks."""
        m, h = self.mfma_floor_s, self.hbm_floor_s
        if m is None or h is None:
            return "unknown"
        return "mfma" if m >= h else "hbm"

    @property
    def floor_s(self) -> float | None:
        m, h = self.mfma_floor_s, self.hbm_floor_s
        if m is None or h is None:
            return None
        return m if m >= h else h

    @property
    def frac(self) -> float | None:
        """Share of the bound pipe's peak the launch achieves (1.0 = at the roofline)."""
        f = self.floor_s
        return None if f is None else f / self.seconds

    @property
    def tflops(self) -> float:
        return self.flops / self.seconds / 1e12

    @property
    def gbs(self) -> float:
        return self.bytes / self.seconds / 1e9

    @property
    def excess_traffic(self) -> float | None:
        """Measured over algorithmic HBM bytes (1.0 = every byte moved once)."""
        return None if self.traffic is None or self.bytes <= 0 else self.traffic / self.bytes

    def bench_fields(self) -> dict:
        """The ``roofline`` object of bench.py's JSON line for this launch."""
        if self.bound == "hbm":
            achieved, peak, unit = self.gbs, self.hbm_peak / 1e9, "GB/s"
        else:
            achieved, peak, unit = self.tflops, (self.mfma_peak or 0.0) / 1e12, "TFLOP/s"
        frac = self.frac
        return {"bound": self.bound, "achieved": round(achieved, 2), "peak": round(peak, 1), "unit": unit,
                "frac": None if frac is None else round(frac, 4), "traffic": self.traffic}

    def to_dict(self) -> dict:
        return {"name": self.name, "precision": self.precision, "flops": self.flops, "bytes": self.bytes,
                "seconds": self.seconds, "tflops": self.tflops, "gbs": self.gbs, "bound": self.bound,
                "frac": self.frac, "traffic": self.traffic, "excess_traffic": self.excess_traffic}


# The reference's name for a roofline point.
RooflinePoint = KernelRoofline


def analyze(name: str, flops: float, bytes_: float, seconds: float, peaks: platform.Peaks | None = None,
            devices: int = 1, peak_flops: float | None = None, *, precision: str = "bf16",
            traffic: float | None = None) -> KernelRoofline:
    """Place one launch on the roofline of ``peaks`` (the attached GPU's when None; no peaks
    off-GPU, so bound 'unknown'). ``precision`` picks the MFMA peak from the MI355X table;
    ``peak_flops`` overrides it (reference signature, src/ferrite/profiling/roofline.py)."""
    if peaks is None:
        peaks = platform.peaks()
    if peaks is None:
        return KernelRoofline(name, float(flops), float(bytes_), float(seconds), precision, traffic)
    if peak_flops is None:
        peak_flops = MI355X_MFMA_PEAKS[precision] if peaks is platform.MI355X else peaks.bf16_flops
    return KernelRoofline(name, float(flops), float(bytes_), float(seconds), precision, traffic,
                          peak_flops * devices, peaks.hbm_bytes_per_s * devices)


def format_table(points: list[KernelRoofline]) -> str:
    """Markdown table: one row per launch, its bound and fraction of that bound's peak."""
    lines = ["| kernel | precision | us | TFLOP/s | GB/s | bound | of peak | traffic / bytes |",
             "|---|---|---:|---:|---:|---|---:|---:|"]
    for p in points:
        frac = "-" if p.frac is None else f"{100 * p.frac:.1f}%"
        ex = "-" if p.excess_traffic is None else f"{p.excess_traffic:.3f}"
        lines.append(f"| {p.name} | {p.precision} | {p.seconds * 1e6:.2f} | {p.tflops:.1f} | {p.gbs:.0f} | "
                     f"{p.bound} | {frac} | {ex} |")
    return "\n".join(lines)
