"""Build libferrite_hip.so (the C ABI of include/ferrite_hip.h) for gfx950.

Each csrc/*.hip file is compiled by hipcc in parallel and the objects are linked
into ferrite/libferrite_hip.so, next to the Python package that loads it. The
library is built in-tree so that it travels with the source tree; nothing is
installed.

    python ferrite-tpu_amd/build_lib.py [--verbose] [--save-temps DIR]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "ferrite", "libferrite_hip.so")
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting packed f32 VALU ops (v_pk_*_f32).
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# Per-source additions. attention.hip: MFMA results in VGPRs rather than AGPRs. The backward's
# softmax gradient reads the S and dP accumulators on the VALU; with AGPR accumulators every
# read is an extra v_accvgpr_read (a quarter of dK/dV's VALU instructions). Measured A/B on one
# MI355X, outputs bitwise equal: dK/dV 166.8 -> 159.9 us at 4x16x2048x128 and 199.7 -> 182.9 us
# at 1x8x8192x64; the forward and dQ kernels (already all-VGPR) are unchanged.
#
# attention.hip also skips the control-flow structurizer on uniform regions. Every branch of the
# attention kernels is wave-uniform (tile counts, parities, row-block bounds), and the
# structurized form of the forward's pipeline tail (the diagonal stage of either parity, the
# one-tile case) kept the accumulators of sibling paths live across each other: the D = 128
# forward needed 256 VGPRs and 12 dwords of scratch per lane, written once per wave (5.5 MiB of
# HBM writes per launch). Without it the same kernel takes 231 VGPRs and no scratch, and every
# attention kernel uses fewer VGPRs. Measured A/B on one MI355X (medians of 7 interleaved
# rounds, outputs bitwise equal): forward 73.5 -> 73.2 us at 4x16x2048x128 and 91.0 -> 91.6 us
# at 1x8x8192x64, dQ with delta 135.6 -> 133.0 us at 1x8x8192x64, the rest unchanged.
#
# attention.hip also raises the size up to which `#pragma unroll` unrolls a loop fully. The D = 256
# forward's stage (48 fragment slots with their DMA and softmax shares) is past the default, and a
# loop left partly rolled indexes the fragment and accumulator arrays at run time, which puts them
# in scratch (2,304 bytes per lane); fully unrolled it keeps them in registers (no scratch). The
# other kernels come out the same.
SOURCE_FLAGS = {
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-structurizecfg-skip-uniform-regions=true",
                      "-mllvm", "-pragma-unroll-threshold=200000"],
}


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the ROCm toolchain is required to build ferrite's HIP kernels")


def _sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, verbose: bool, save_temps: str | None) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    cwd = None
    if save_temps:  # temporaries (including the gfx950 .s) land in the working directory
        os.makedirs(save_temps, exist_ok=True)
        cmd.append("-save-temps")
        cwd = save_temps
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True, cwd=cwd)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; that is harmless.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False, save_temps: str | None = None) -> str:
    """Compile every csrc/*.hip for gfx950 and link ferrite/libferrite_hip.so. Returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = _sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, save_temps), srcs))
    tmp = OUT + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--save-temps", default=None, help="directory for compiler temporaries (ISA)")
    a = ap.parse_args(argv)
    print(build(a.verbose, a.save_temps))


if __name__ == "__main__":
    main()
