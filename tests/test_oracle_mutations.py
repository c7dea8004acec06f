"""Plants plausible mistakes in the CPU oracle and checks that its pinning tests catch them.

Each mutation replaces one oracle function (monkeypatch, CPU only) with a variant carrying a
typical slip -- a dropped factor, a transposed operand, an off-by-one index, a wrong sign --
and runs the test of tests/test_oracle.py that is meant to catch it; the test must fail.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import field_oracle as fo
from tests import test_oracle as t


def _basis_no_half(coords, mu, inv_cov, det_cov, normalize, clamp_quad):
    diff = coords.unsqueeze(0) - mu.unsqueeze(1)
    quad = torch.einsum("kmd,kde,kme->km", diff, inv_cov, diff)
    if clamp_quad is not None:
        quad = quad.clamp(min=0.0, max=clamp_quad)
    return torch.exp(-quad)  # missing the 1/2


def _basis_swapped_axes(coords, mu, inv_cov, det_cov, normalize, clamp_quad):
    return _ORIG_BASIS(coords.flip(-1), mu, inv_cov, det_cov, normalize, clamp_quad)


def _basis_norm_without_sqrt(coords, mu, inv_cov, det_cov, normalize, clamp_quad):
    b = _ORIG_BASIS(coords, mu, inv_cov, det_cov, False, clamp_quad)
    if normalize:
        b = b * (1.0 / (2.0 * math.pi * det_cov.clamp_min(torch.finfo(coords.dtype).eps))).unsqueeze(-1)
    return b


def _activate_no_eps(chol_raw, eps=fo.CHOLESKY_EPS):
    return _ORIG_ACTIVATE(chol_raw, 0.0)


def _activate_l21_upper(chol_raw, eps=fo.CHOLESKY_EPS):
    L = _ORIG_ACTIVATE(chol_raw, eps)
    return L.transpose(-1, -2).contiguous()  # upper instead of lower factor


def _bounds_m_not_m1(mu, chol, M, N, to, ti, sigma):
    b = _ORIG_BOUNDS(mu, chol, M + 1, N + 1, to, ti, sigma)  # (mu+1)/2 * M instead of * (M-1)
    R, C = (M + to - 1) // to, (N + ti - 1) // ti
    clip = lambda x, hi: x.clamp(0, hi)  # noqa: E731
    tr0, tr1, tc0, tc1 = clip(b.tile_r0, R - 1), clip(b.tile_r1, R - 1), clip(b.tile_c0, C - 1), clip(b.tile_c1, C - 1)
    return fo.TileBounds(tr0, tr1, tc0, tc1, (tr1 - tr0 + 1) * (tc1 - tc0 + 1), R, C)


def _bounds_tile_ceil(mu, chol, M, N, to, ti, sigma):
    b = _ORIG_BOUNDS(mu, chol, M, N, to, ti, sigma)
    tr1 = (b.tile_r1 + 1).clamp(max=b.num_tile_rows - 1)  # last tile one too far
    return fo.TileBounds(b.tile_r0, tr1, b.tile_c0, b.tile_c1,
                         (tr1 - b.tile_r0 + 1) * (b.tile_c1 - b.tile_c0 + 1), b.num_tile_rows,
                         b.num_tile_cols)


def _index_descending(b):
    idx = _ORIG_INDEX(b)
    ids = idx.gaussian_ids.clone()
    ptr = idx.tile_ptr.tolist()
    for s, e in zip(ptr[:-1], ptr[1:]):
        ids[s:e] = ids[s:e].flip(0)
    return fo.TileIndex(idx.tile_ptr, ids, idx.tile_ids, idx.num_tile_rows, idx.num_tile_cols)


_ORIG_BASIS = fo._basis
_ORIG_ACTIVATE = fo.activate_cholesky
_ORIG_BOUNDS = fo.tile_bounds
_ORIG_INDEX = fo.build_tile_index

MUTATIONS = [
    ("_basis", _basis_no_half, lambda: t.test_render_single_gaussian_closed_form(False, 80.0)),
    ("_basis", _basis_swapped_axes, lambda: t.test_render_single_gaussian_closed_form(False, 80.0)),
    ("_basis", _basis_norm_without_sqrt, lambda: t.test_render_single_gaussian_closed_form(True, 80.0)),
    ("activate_cholesky", _activate_no_eps, t.test_activate_cholesky_against_float64_softplus),
    ("activate_cholesky", _activate_l21_upper, t.test_activate_cholesky_against_float64_softplus),
    ("tile_bounds", _bounds_m_not_m1, t.test_tile_bounds_against_float64),
    ("tile_bounds", _bounds_tile_ceil, t.test_tile_bounds_centred_isotropic),
    ("build_tile_index", _index_descending, lambda: t.test_golden_tiny_ragged()),
]


@pytest.mark.parametrize("attr,mutant,check", MUTATIONS,
                         ids=[m[1].__name__.lstrip("_") for m in MUTATIONS])
def test_planted_mistake_is_caught(monkeypatch, attr, mutant, check):
    monkeypatch.setattr(fo, attr, mutant)
    with pytest.raises(AssertionError):
        check()


def test_unmutated_checks_pass():
    for _, _, check in MUTATIONS:
        check()
