"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

The reference's own tests hold no fixtures for this path, so these are produced by the oracle
(oracle/field_oracle.py) after the oracle has been pinned by the closed-form, brute-force and
gradcheck tests in tests/test_oracle.py.  They freeze its outputs -- bit-exact binning, the
fp32 field and the gradients -- so that a change of torch version or host C library on another
machine (which would change the oracle's CPU arithmetic) is caught, and so that GPU tests have
fixed expected values.  Every file records the torch version it was written with.

Files (numpy .npz, no pickles):
  tiny_ragged.npz   45x70 field, K=12, 16x16 tiles (ragged last tile row and column): inputs,
                    delta, tile_ptr, gaussian ids, d_mu, d_chol_raw, d_amp
  cfg1_seed0.npz    BASELINE cfg1 (320x320, K=64): inputs except coords (linspace), binning,
                    gradients, and delta at 2048 fixed positions plus its sum / sum of squares
  softplus.npz      F.softplus of strided views on boundary inputs (bit patterns in and out)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from guass_amd import workloads as wl  # noqa: E402
from oracle import field_oracle as fo  # noqa: E402

TILE, SIGMA, CLAMP = 16, 3.0, 80.0


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy()


def tiny_ragged() -> dict:
    p = wl.make_problem("tiny_ragged", 45, 70, 12, np.log(3.0), 0.6, seed=11)
    out = fo.gaussian_field_fwd_bwd(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad,
                                    TILE, TILE, SIGMA, False, CLAMP)
    delta, tile_ptr, ids, d_mu, d_raw, d_amp = out
    return {"out_features": np.int64(45), "in_features": np.int64(70),
            "row_coords": _np(p.row_coords), "col_coords": _np(p.col_coords), "mu": _np(p.mu),
            "chol_raw": _np(p.chol_raw), "amp": _np(p.amp), "grad": _np(p.grad),
            "delta": _np(delta), "tile_ptr": _np(tile_ptr), "gaussian_ids": _np(ids),
            "d_mu": _np(d_mu), "d_chol_raw": _np(d_raw), "d_amp": _np(d_amp)}


def cfg1() -> dict:
    p = wl.cfg1(0)
    delta, tile_ptr, ids, d_mu, d_raw, d_amp = fo.gaussian_field_fwd_bwd(
        p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, TILE, TILE, SIGMA, False, CLAMP)
    g = torch.Generator().manual_seed(1234)
    pos = torch.randperm(delta.numel(), generator=g)[:2048].sort().values
    d64 = delta.to(torch.float64)
    return {"out_features": np.int64(320), "in_features": np.int64(320), "mu": _np(p.mu),
            "chol_raw": _np(p.chol_raw), "amp": _np(p.amp), "grad_seed": np.int64(0),
            "tile_ptr": _np(tile_ptr), "gaussian_ids": _np(ids).astype(np.int32),
            "delta_positions": _np(pos).astype(np.int32), "delta_values": _np(delta[pos]),
            "delta_sum": np.float64(d64.sum()), "delta_sumsq": np.float64((d64 * d64).sum()),
            "d_mu": _np(d_mu), "d_chol_raw": _np(d_raw), "d_amp": _np(d_amp)}


def softplus_vectors() -> dict:
    bits = [0x00000000, 0x80000000, 0x00000001, 0x007fffff, 0x00800000, 0x3f800000, 0xbf800000,
            0x41a00000, 0x41a00001, 0x419fffff, 0xc1a00000, 0xc2cf0000, 0xc2d00000, 0xc2d00001,
            0xc2aeac4f, 0xc2aeac50, 0xc2b00000, 0xc2c00000, 0x3ed413d7, 0x3ed413d6, 0x31000000,
            0x24800000, 0xbe95f61f, 0x3504f7ff, 0x7f7fffff, 0xff7fffff, 0x7f800000, 0xff800000,
            0xc27c65d9, 0x42b17218, 0x42b17217, 0xc2b17218]
    g = torch.Generator().manual_seed(99)
    rnd = torch.randint(0, 2**32, (4096,), generator=g, dtype=torch.int64)
    rnd = rnd[((rnd >> 23) & 0xFF) != 0xFF]  # finite
    xb = torch.cat((torch.tensor(bits, dtype=torch.int64), rnd)).to(torch.int64)
    x = torch.from_numpy(xb.numpy().astype(np.uint32).view(np.float32).copy())
    # strided column view, as activate_cholesky applies softplus (covariance.py:23,25)
    host = torch.zeros(x.numel(), 3, dtype=torch.float32)
    host[:, 0] = x
    y = torch.nn.functional.softplus(host[:, 0])
    return {"x_bits": x.numpy().view(np.uint32).copy(), "y_bits": y.numpy().view(np.uint32).copy()}


def main() -> None:
    meta = {"torch_version": np.array(torch.__version__)}
    for name, fn in (("tiny_ragged", tiny_ragged), ("cfg1_seed0", cfg1), ("softplus", softplus_vectors)):
        data = fn()
        data.update(meta)
        np.savez_compressed(HERE / f"{name}.npz", **data)
        print(f"wrote {name}.npz ({(HERE / f'{name}.npz').stat().st_size} bytes)")


if __name__ == "__main__":
    main()
