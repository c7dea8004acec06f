"""Parity assertions shared by the GPU tests (bars from BASELINE.json's north star).

* binning (tile_ptr, gaussian ids): bit-exact;
* delta-W: max |delta - ref| <= 1e-5 * max |ref|  (element-wise relative error is ill-posed
  near the zeros of a signed sum of Gaussians, so the scale is the field's peak);
* gradients: ||g - ref|| / ||ref|| <= 1e-4 per tensor, and element-wise
  |g - ref| <= 1e-4 * max|ref| + 1e-3 * |ref|.
"""

from __future__ import annotations

import torch

FWD_RTOL = 1e-5
GRAD_RTOL = 1e-4

# A tile of more than this many Gaussians is a heavy tile (the library's kHeavyTile): where a
# single field launches heavy-tile workgroups, four waves share such a tile and their partial sums
# are added in a different order from one wave's.
HEAVY_TILE = 24

# Order-independent checksum of F.softplus over all 2^32 fp32 inputs, computed from the host C
# library by oracle/libm_sweep.c; the GPU self-test (gf_selftest_softplus) must reproduce it.
SOFTPLUS_CHECKSUM = 0x06C0D4E444E1424F


def binning_equal(tile_ptr, ids, tile_ptr_ref, ids_ref) -> None:
    tp = tile_ptr.detach().cpu().to(torch.int64)
    gi = ids.detach().cpu().to(torch.int64)
    assert tp.shape == tile_ptr_ref.shape, (tp.shape, tile_ptr_ref.shape)
    assert torch.equal(tp, tile_ptr_ref), "tile_ptr differs"
    assert gi.shape == ids_ref.shape, (gi.shape, ids_ref.shape)
    if not torch.equal(gi, ids_ref):
        bad = (gi != ids_ref).nonzero()[:5].flatten().tolist()
        raise AssertionError(f"gaussian_ids_sorted differs at {bad}")


def field_close(delta, ref, rtol: float = FWD_RTOL) -> float:
    d = delta.detach().cpu().reshape(-1).to(torch.float64)
    r = ref.detach().cpu().reshape(-1).to(torch.float64)
    scale = float(r.abs().max()) if r.numel() else 0.0
    err = float((d - r).abs().max()) if r.numel() else 0.0
    assert err <= rtol * scale + 1e-30, f"delta max err {err:.3e} > {rtol} * {scale:.3e}"
    return err / scale if scale > 0 else 0.0


def grad_close(g, ref, name: str, rtol: float = GRAD_RTOL) -> float:
    a = g.detach().cpu().reshape(-1).to(torch.float64)
    b = ref.detach().cpu().reshape(-1).to(torch.float64)
    nb = float(b.norm())
    rel = float((a - b).norm()) / nb if nb > 0 else float((a - b).norm())
    assert rel <= rtol, f"{name}: norm-relative error {rel:.3e} > {rtol}"
    if b.numel():
        tol = 1e-4 * float(b.abs().max()) + 1e-3 * b.abs()
        worst = float(((a - b).abs() - tol).max())
        assert worst <= 0.0, f"{name}: element-wise error exceeds bound by {worst:.3e}"
    return rel
