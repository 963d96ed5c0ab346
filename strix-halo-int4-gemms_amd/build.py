"""Builds libamd_strix_halo_kernels_gfx950.so (HIP kernels + C ABI) in-tree.

The library is compiled from csrc/ with hipcc for gfx950 only and written next
to the Python package (amd_strix_halo_kernels/), where the ctypes bridge loads
it.  Every translation unit is compiled in parallel; objects go to _build/.

    python build.py [--jobs N]
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
PACKAGE = ROOT / "amd_strix_halo_kernels"
LIBRARY_NAME = "libamd_strix_halo_kernels_gfx950.so"
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for every kernel; contraction is off
# so epilogue products round exactly like the reference's separate multiplies.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc was not found; ROCm is required to build the gfx950 kernels")
    return path


# The direct-to-LDS dense objects hold 256 accumulators per lane; the
# iterative ILP machine scheduler keeps them in place in AGPRs, where the
# default scheduler's allocation rotates them through copies every K step.
DMA_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]


def translation_units() -> list[tuple[str, Path, list[str]]]:
    units: list[tuple[str, Path, list[str]]] = []
    for bits in (4, 8):
        for layout in (0, 1, 2):
            defs = [f"-DSHK_BITS={bits}", f"-DSHK_LAYOUT={layout}"]
            units.append((f"dense_dma_{bits}_{layout}", CSRC / "k_dense.hip", [*defs, "-DSHK_DENSE_DMA=1", *DMA_FLAGS]))
            units.append((f"dense_{bits}_{layout}", CSRC / "k_dense.hip", [*defs, "-DSHK_DENSE_DMA=0"]))
    # fp6 path: the GEMM keeps 256 accumulators like the DMA objects; the
    # operand conversion is compiled with the default scheduler.
    units.append(("dense_f6", CSRC / "k_f6.hip", list(DMA_FLAGS)))
    units.append(("f6pack", CSRC / "k_f6pack.hip", []))
    units.append(("ragged_f6", CSRC / "k_f6ragged.hip", list(DMA_FLAGS)))
    units.append(("quant", CSRC / "k_quant.hip", []))
    for layout in (0, 1, 2, 3):
        units.append((f"ragged_{layout}", CSRC / "k_ragged.hip", [f"-DSHK_LAYOUT={layout}"]))
    for bits in (4, 8):
        for layout in (0, 1, 2):
            units.append((f"skinny_{bits}_{layout}", CSRC / "k_skinny.hip", [f"-DSHK_BITS={bits}", f"-DSHK_LAYOUT={layout}"]))
    units.append(("capi", CSRC / "capi.hip", []))
    return units


def _compile(unit: tuple[str, Path, list[str]]) -> tuple[str, float, str]:
    name, src, defines = unit
    obj = BUILD / f"{name}.o"
    cmd = [hipcc(), *HIP_FLAGS, *defines, "-c", str(src), "-o", str(obj)]
    t0 = time.time()
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compiling {name} failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return name, time.time() - t0, str(obj)


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    units = translation_units()
    jobs = jobs or min(len(units), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    t0 = time.time()
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_compile, units))
    if verbose:
        for name, secs, _ in results:
            print(f"  compiled {name:12s} {secs:6.1f}s", flush=True)
    objects = [obj for _, _, obj in results]
    out = PACKAGE / LIBRARY_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} in {time.time() - t0:.1f}s", flush=True)
    return out


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=None)
    args = parser.parse_args(argv)
    build(args.jobs)
    return 0


if __name__ == "__main__":
    sys.exit(main())
