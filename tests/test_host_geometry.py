"""The binning arithmetic the gfx950 kernels run, built for the host, against the oracle (CPU).

libgaussfield_host.so compiles the same headers as the kernels (guass_amd/csrc/geometry.h,
libm_f32.h) with g++ and no FP contraction.  These tests pin them bit for bit:

* softplus (covariance.py:23,25): exhaustively against the host C library over all 2^32 fp32
  inputs -- whose checksum the GPU self-test reproduces -- and on samples against
  F.softplus of strided views, which is what the reference CPU path calls;
* activated Cholesky factor and fp32 covariance (covariance.py:14-38, bounds.py:40-41);
* tile rectangles (bounds.py:24-75) on the BASELINE configurations.
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from guass_amd import workloads as wl
from oracle import field_oracle as fo
from tests.parity import SOFTPLUS_CHECKSUM

ROOT = Path(__file__).resolve().parent.parent
HOST_LIB = Path(os.environ.get("GUASS_AMD_HOST_LIB") or ROOT / "guass_amd" / "libgaussfield_host.so")
SWEEP = ROOT / "oracle" / "_build" / "libm_sweep"
_P = ctypes.c_void_p
_I = ctypes.c_int64


@pytest.fixture(scope="module")
def host():
    if not HOST_LIB.exists():
        pytest.fail(f"{HOST_LIB} is not built (python -m guass_amd.build)")
    lib = ctypes.CDLL(str(HOST_LIB))
    lib.gfh_softplus.argtypes = [_P, _P, _I]
    lib.gfh_tile_rects.argtypes = [_I, _P, _P, _I, _I, _I, _I, ctypes.c_double, _P, _P]
    lib.gfh_chol_cov.argtypes = [_I, _P, _P, _P]
    return lib


def _softplus_host(lib, x: torch.Tensor) -> torch.Tensor:
    x = x.contiguous()
    y = torch.empty_like(x)
    lib.gfh_softplus(x.data_ptr(), y.data_ptr(), x.numel())
    return y


def test_softplus_matches_torch_strided(host):
    g = torch.Generator().manual_seed(1)
    bits = torch.randint(0, 2**32, (1 << 20,), generator=g, dtype=torch.int64)
    x = torch.from_numpy(bits.numpy().astype(np.uint32).view(np.float32).copy())
    x = torch.cat((x, torch.linspace(-110.0, 30.0, 200001)))
    col = torch.zeros(x.numel(), 3)
    col[:, 0] = x
    ref = F.softplus(col[:, 0])  # strided view, as activate_cholesky applies it
    got = _softplus_host(host, x)
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(torch.int32), ref[~nan].view(torch.int32))


def test_softplus_exhaustive_against_host_libm():
    """All 2^32 inputs (about 45 s on 8 cores); prints the checksum the GPU must reproduce."""
    if not SWEEP.exists():
        pytest.fail(f"{SWEEP} is not built (python -m guass_amd.build)")
    out = subprocess.run([str(SWEEP), "1"], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    m = re.search(r"softplus_checksum=0x([0-9a-f]+)", out.stdout)
    assert m and int(m.group(1), 16) == SOFTPLUS_CHECKSUM, out.stdout


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3", "cfg5", "cfg5c"])
def test_cholesky_and_covariance_bit_exact(host, cfg):
    p = wl.CONFIGS[cfg](0, with_grad=False)
    K = p.k
    chol = torch.empty(K, 3)
    cov = torch.empty(K, 3)
    host.gfh_chol_cov(K, p.chol_raw.data_ptr(), chol.data_ptr(), cov.data_ptr())
    L = fo.activate_cholesky(p.chol_raw)
    S = L @ L.transpose(-1, -2)  # the reference's fp32 batched product (bounds.py:40)
    assert torch.equal(chol, torch.stack((L[:, 0, 0], L[:, 1, 0], L[:, 1, 1]), 1))
    assert torch.equal(cov, torch.stack((S[:, 0, 0], S[:, 0, 1], S[:, 1, 1]), 1))


@pytest.mark.parametrize("cfg,seeds", [("cfg1", 8), ("cfg2", 8), ("cfg3", 4), ("cfg5", 3), ("cfg5c", 2)])
@pytest.mark.parametrize("tiles,sigma", [((16, 16), 3.0), ((8, 24), 2.5)])
def test_tile_rects_bit_exact(host, cfg, seeds, tiles, sigma):
    for seed in range(seeds):
        p = wl.CONFIGS[cfg](seed, with_grad=False)
        K = p.k
        rects = torch.empty(K, 4, dtype=torch.int64)
        touched = torch.empty(K, dtype=torch.int64)
        host.gfh_tile_rects(K, p.mu.data_ptr(), p.chol_raw.data_ptr(), p.out_features,
                            p.in_features, tiles[0], tiles[1], sigma, rects.data_ptr(),
                            touched.data_ptr())
        b = fo.tile_bounds(p.mu, fo.activate_cholesky(p.chol_raw), p.out_features, p.in_features,
                           tiles[0], tiles[1], sigma)
        ref = torch.stack((b.tile_r0, b.tile_r1, b.tile_c0, b.tile_c1), 1)
        assert torch.equal(rects, ref), f"{cfg} seed {seed}"
        assert torch.equal(touched, b.tiles_touched)
