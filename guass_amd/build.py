"""Builds the native libraries in-tree.

* ``guass_amd/libgaussfield.so``       gfx950 kernels + C ABI (hipcc, --offload-arch=gfx950)
* ``guass_amd/libgaussfield_host.so``  host build of the per-Gaussian geometry (g++), used by
                                       CPU tests to pin the exact arithmetic the GPU runs
* ``oracle/_build/libm_sweep``         exhaustive libm check (test infrastructure)

``python -m guass_amd.build`` builds all three; ``build_all()`` is what ``__graft_entry__.build``
calls.  Every call compiles (no up-to-date check), so a stale library is never picked up.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libgaussfield.so"
HOST_LIB = PKG / "libgaussfield_host.so"

# Packed FP32 instructions are disabled on this pool (-packed-fp32-ops); fp32 denormals are kept
# (the bit-exact softplus path passes through subnormal expf results).
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-flush-denormals-to-zero",
    "-mcode-object-version=5",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build_gpu_lib() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, str(CSRC / "gaussfield.hip"), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build_host_lib() -> Path:
    tmp = HOST_LIB.with_suffix(".so.tmp")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
          str(CSRC / "host_geometry.cpp"), "-o", str(tmp)])
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build_oracle_tools() -> Path:
    out = ROOT / "oracle" / "_build"
    out.mkdir(exist_ok=True)
    exe = out / "libm_sweep"
    _run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", str(ROOT / "oracle" / "libm_sweep.c"),
          "-o", str(exe), "-lm"])
    return exe


def build_all(verbose: bool = True) -> None:
    for fn in (build_gpu_lib, build_host_lib, build_oracle_tools):
        path = fn()
        if verbose:
            print(f"[guass_amd.build] built {path.relative_to(ROOT)}", flush=True)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
