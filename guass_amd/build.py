"""Builds the native libraries in-tree.

* ``guass_amd/libgaussfield.so``       gfx950 kernels + C ABI (hipcc, --offload-arch=gfx950)
* ``guass_amd/libgaussfield_host.so``  host build of the per-Gaussian geometry (g++), used by
                                       CPU tests to pin the exact arithmetic the GPU runs
* ``oracle/_build/libm_sweep``         exhaustive libm check (test infrastructure)
* ``_build/sanitize/``                 (``build_sanitized``, for the CPU tests) both libraries with
                                       their host code under ASan + UBSan

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


SANITIZE_DIR = ROOT / "_build" / "sanitize"
SANITIZE_FLAGS = ["-fsanitize=address", "-fsanitize=undefined", "-fno-omit-frame-pointer"]


def clangxx() -> str:
    """The clang++ of the ROCm toolchain (hipcc's host compiler, whose sanitizer runtime the
    host-sanitized builds link against)."""
    for cand in ("/opt/rocm/llvm/bin/clang++", shutil.which("amdclang++")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("the ROCm clang++ was not found")


def asan_runtime() -> Path:
    """The shared AddressSanitizer runtime (with the UndefinedBehaviorSanitizer handlers) that a
    process must preload to load the host-sanitized libraries."""
    out = subprocess.run([clangxx(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                         text=True, check=True).stdout.strip()
    path = Path(out)
    if not path.is_file():
        raise RuntimeError(f"no shared ASan runtime at {out}")
    return path


def build_sanitized(out_dir: Path = SANITIZE_DIR) -> dict[str, Path]:
    """Both native libraries with their HOST code under AddressSanitizer and
    UndefinedBehaviorSanitizer (-O1 -g): the C ABI's argument checks, layout and block-map
    arithmetic (gf_batch_plan) and the host geometry build.  The gfx950 device code is compiled
    as usual (each -fsanitize= reaches the host compilation only, through -Xarch_host).  Load them
    with asan_runtime() preloaded and GUASS_AMD_LIB pointing at the library."""
    out_dir.mkdir(parents=True, exist_ok=True)
    lib, host = out_dir / "libgaussfield.so", out_dir / "libgaussfield_host.so"
    hip = [f for f in HIP_FLAGS if f != "-O3"] + ["-O1", "-g"]
    host_only = [a for f in SANITIZE_FLAGS for a in ("-Xarch_host", f)]
    _run([hipcc(), *hip, *host_only, str(CSRC / "gaussfield.hip"), "-o", str(lib)])
    _run([clangxx(), "-O1", "-g", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", *SANITIZE_FLAGS,
          str(CSRC / "host_geometry.cpp"), "-o", str(host)])
    return {"lib": lib, "host_lib": host}


def build_all(verbose: bool = True) -> None:
    for fn in (build_gpu_lib, build_host_lib, build_oracle_tools):
        path = fn()
        if verbose:
            print(f"[guass_amd.build] built {path.relative_to(ROOT)}", flush=True)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
