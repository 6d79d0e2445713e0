"""Build libvsplat.so (the gfx950 kernels and the C ABI) in-tree.

    python -m vauss_amd.build          # compile every source, in parallel
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = ROOT / "_build" / "vsplat"
LIB = PKG / "libvsplat.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -ffp-contract=off: every multiply-add is fused only where the source writes
# an fma, which the bit-exact parity of projection, binning and compositing
# relies on.  Packed-FP32 generation is switched off for all kernels.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    "-I", str(ROOT / "include"),
]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-fno-gpu-rdc", "-munsafe-fp-atomics"]

SOURCES = ["k_project.hip", "k_project_bwd.hip", "k_project_update.hip", "k_raster.hip", "k_loss.hip", "k_sh_step.hip", "k_pose.hip", "k_neural.hip",
           "k_scan.hip", "k_sort.hip", "k_calib.hip", "api.hip", "camera.cpp"]
HEADERS = ["vs_device.h", "vs_camera.h", "vs_sh.h", "vs_vjp.h", "vs_adam.h", "vs_neural.h", "vs_surfel.h",
           "vs_internal.h"]


def _compile(src: str) -> Path:
    out = OBJ / (src + ".o")
    is_hip = src.endswith(".hip")
    cmd = [HIPCC, *COMMON, *(DEVICE if is_hip else []), "-x", "hip" if is_hip else "c++", "-c",
           str(CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return out


def build(verbose: bool = True) -> Path:
    """Compile every source for gfx950 and link vauss_amd/libvsplat.so."""
    OBJ.mkdir(parents=True, exist_ok=True)
    jobs = min(len(SOURCES), max(1, min(16, os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


def build_oracle(verbose: bool = True) -> None:
    """Compile the CPU oracle (test infrastructure) with its own Makefile."""
    res = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    if verbose:
        print("built oracle/liboracle.so", file=sys.stderr)


if __name__ == "__main__":
    build()
