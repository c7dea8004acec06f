"""The CPU tests of the native libraries with their host code under AddressSanitizer and
UndefinedBehaviorSanitizer.

The host side of libgaussfield.so -- argument checks, workspace layouts, tile grids, the batch
plan's offsets and block maps (gf_batch_plan), the allocation-free entry's limits, the fused
entry's refusals -- and the host geometry build (libgaussfield_host.so) are compiled with
-fsanitize=address,undefined (guass_amd.build.build_sanitized; the gfx950 device code as usual)
and the CPU tests that call them run in a child process with the sanitizer runtime preloaded.
Any sanitizer report fails the run (halt_on_error / abort_on_error).
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

from guass_amd import build

ROOT = Path(__file__).resolve().parent.parent
NATIVE_TESTS = ["tests/test_abi.py", "tests/test_host_geometry.py", "tests/test_zz_no_alloc.py",
                "tests/test_layers.py", "tests/test_capture_sequence.py"]


@pytest.fixture(scope="module")
def libs():
    """Both libraries built once for this module (host code under ASan + UBSan)."""
    return build.build_sanitized()


def test_native_cpu_tests_under_asan_and_ubsan(libs):
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": str(build.asan_runtime()),
        # Python and torch are not instrumented: their allocations at exit are not this code's leaks
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:halt_on_error=1:symbolize=1",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "GUASS_AMD_LIB": str(libs["lib"]),
        "GUASS_AMD_HOST_LIB": str(libs["host_lib"]),
    })
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                           *NATIVE_TESTS], cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = proc.stdout[-6000:] + "\n" + proc.stderr[-6000:]
    assert proc.returncode == 0, out
    for marker in ("ERROR: AddressSanitizer", "runtime error:", "SUMMARY: UndefinedBehaviorSanitizer"):
        assert marker not in proc.stdout + proc.stderr, out
    assert " passed" in proc.stdout, out


PROBE = """
import ctypes, torch
from guass_amd import _native as N
L = N.lib()
cfg = N.make_config(16, 16, 3.0, False, 80.0)
n = 8  # a table past pymalloc's small-object size, so that it comes from malloc (with redzones)
tab = (N.GfLayer * n)()
for ly in tab:
    ly.out_features, ly.in_features, ly.k = 64, 64, 4
    for f in ("row_coords", "col_coords", "mu", "chol_raw", "amp", "delta", "tile_ptr", "num_pairs",
              "forward_workspace"):
        setattr(ly, f, 4096)  # never dereferenced: a size query
    ly.forward_workspace_bytes = 1 << 30
info = N.GfBatchInfo()
assert L.gf_batch_plan(ctypes.byref(cfg), tab, n, None, 0, ctypes.byref(info), None) == 0
L.gf_batch_plan(ctypes.byref(cfg), tab, n + 1, None, 0, ctypes.byref(info), None)  # one layer too many
"""


def test_sanitizer_reports_a_host_overflow(libs):
    """The harness is live: a caller's error that makes the library's host code read past the
    caller's layer table (n_layers one larger than the table) is reported by ASan in the
    sanitized build.  Host memory only; no device work (a size query)."""
    env = dict(os.environ)
    env.update({"LD_PRELOAD": str(build.asan_runtime()), "ASAN_OPTIONS": "detect_leaks=0",
                "GUASS_AMD_LIB": str(libs["lib"])})
    proc = subprocess.run([sys.executable, "-c", PROBE], cwd=ROOT, env=env, capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode != 0
    assert "AddressSanitizer: heap-buffer-overflow" in proc.stderr and "gf_batch_plan" in proc.stderr, \
        proc.stderr[-3000:]
