"""Pins the CPU oracle (oracle/field_oracle.py) without importing the reference.

The reference's tests hold no golden vectors for this path, so each oracle function is checked
against what the mathematics fixes, chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails at least one check:

* activate_cholesky (covariance.py:14-26)    float64 softplus; layout of L
* tile_bounds       (bounds.py:24-75)         closed-form boxes (centred, corner, huge, tiny,
                                              ragged) and a float64 recomputation
* build_tile_index  (tile_index.py:51-99)     brute-force enumeration of every tile
* render_tiles      (tile_accumulate.py:95-131, gaussian_core.py:55-82)
                                              closed-form single Gaussian (with clamp and
                                              normalisation), linearity, superposition, the
                                              dense field within the 3-sigma truncation bound
* backward (autograd through the same program, backward.cu:541-716)
                                              fp64 gradcheck, closed-form d_amp, closed-form
                                              isotropic d_mu, closed-form covariance chain
* batched / fp64 variants                     agree with the per-tile loop
* golden fixtures (tests/golden)              reproduced bit for bit (binning) or to fp32
                                              rounding (field, gradients)
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from guass_amd import workloads as wl
from oracle import field_oracle as fo

GOLDEN = Path(__file__).resolve().parent / "golden"
E45 = math.exp(-4.5)


def _chol_raw_for(l11: float, l21: float, l22: float) -> torch.Tensor:
    """chol_raw whose activated factor is (close to) the given one."""
    inv = lambda y: math.log(math.expm1(y - fo.CHOLESKY_EPS))  # noqa: E731
    return torch.tensor([[inv(l11), l21, inv(l22)]], dtype=torch.float32)


def _exact_field(rc, cc, mu, chol, amp, normalize=False, clamp=80.0):
    """float64 closed form amp * exp(-q/2) [/ (2 pi sqrt det)] at every pixel, per Gaussian."""
    rc64, cc64 = rc.to(torch.float64), cc.to(torch.float64)
    L = chol.to(torch.float64)
    cov = L @ L.transpose(-1, -2)
    out = []
    for g in range(mu.shape[0]):
        a, b, d = cov[g, 0, 0], cov[g, 0, 1], cov[g, 1, 1]
        det = a * d - b * b
        dx = (rc64 - float(mu[g, 0])).reshape(-1, 1)
        dy = (cc64 - float(mu[g, 1])).reshape(1, -1)
        q = (d * dx * dx - 2.0 * b * dx * dy + a * dy * dy) / det
        if clamp is not None:
            q = q.clamp(0.0, clamp)
        v = float(amp[g, 0]) * torch.exp(-0.5 * q)
        if normalize:
            v = v / (2.0 * math.pi * max(math.sqrt(float(det)), torch.finfo(torch.float32).eps))
        out.append(v)
    return torch.stack(out)  # [K, M, N]


def _tile_mask(b: fo.TileBounds, g: int, M: int, N: int, to: int, ti: int) -> torch.Tensor:
    rows = torch.arange(M) // to
    cols = torch.arange(N) // ti
    rm = (rows >= int(b.tile_r0[g])) & (rows <= int(b.tile_r1[g]))
    cm = (cols >= int(b.tile_c0[g])) & (cols <= int(b.tile_c1[g]))
    return rm.reshape(-1, 1) & cm.reshape(1, -1)


# ------------------------------------------------------------------------------ covariance


def test_activate_cholesky_against_float64_softplus():
    g = torch.Generator().manual_seed(0)
    raw = torch.cat((torch.randn(2000, 3, generator=g) * 8.0,
                     torch.tensor([[20.0, 1.5, 20.5], [-30.0, -2.0, 25.0], [0.0, 0.0, -88.0]])))
    L = fo.activate_cholesky(raw)
    assert L.shape == (raw.shape[0], 2, 2)
    assert torch.all(L[:, 0, 1] == 0)
    assert torch.equal(L[:, 1, 0], raw[:, 1])
    for col, (i, j) in ((0, (0, 0)), (2, (1, 1))):
        x = raw[:, col].to(torch.float64)
        sp = torch.where(x > 20.0, x, torch.log1p(torch.exp(x)))
        want = (sp.to(torch.float32) + torch.tensor(fo.CHOLESKY_EPS, dtype=torch.float32))
        got = L[:, i, j]
        ulp = torch.abs(want) * 2.0**-23 + 1e-45
        assert torch.all((got - want).abs() <= 2 * ulp), "softplus(x) + eps off by more than 2 ulp"
        big = raw[:, col] > 20.0
        assert torch.equal(got[big], raw[big, col] + fo.CHOLESKY_EPS)  # threshold branch: x itself


def test_softplus_golden_bits():
    d = np.load(GOLDEN / "softplus.npz")
    x = torch.from_numpy(d["x_bits"].view(np.float32).copy())
    raw = torch.zeros(x.numel(), 3)
    raw[:, 0] = x
    raw[:, 2] = x
    L = fo.activate_cholesky(raw, eps=0.0)
    got = L[:, 0, 0].numpy().view(np.uint32)
    want = d["y_bits"]
    nan = np.isnan(want.view(np.float32))
    assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(got.view(np.float32)[nan]).all()


# ------------------------------------------------------------------------------ tile bounds


def _bounds(mu, raw, M, N, to=16, ti=16, sigma=3.0):
    return fo.tile_bounds(mu, fo.activate_cholesky(raw), M, N, to, ti, sigma)


def test_tile_bounds_centred_isotropic():
    M = N = 161  # centre pixel 80 exactly
    for s in (0.011, 0.0512, 0.13, 0.31):
        b = _bounds(torch.zeros(1, 2), _chol_raw_for(s, 0.0, s), M, N)
        L = fo.activate_cholesky(_chol_raw_for(s, 0.0, s))
        std = float(L[0, 0, 0])
        half = 3.0 * std * 0.5 * (M - 1)
        lo, hi = math.floor(80.0 - half), math.ceil(80.0 + half)
        assert abs(half - round(half)) > 1e-3
        lo, hi = max(lo, 0), min(hi, M - 1)
        want = (lo // 16, hi // 16)
        assert (int(b.tile_r0), int(b.tile_r1)) == want
        assert (int(b.tile_c0), int(b.tile_c1)) == want
        assert int(b.tiles_touched) == (want[1] - want[0] + 1) ** 2


def test_tile_bounds_corner_huge_tiny_ragged():
    M, N = 45, 70  # 3 x 5 tiles, last row 13 px, last column 6 px
    mu = torch.tensor([[-1.0, -1.0], [1.0, 1.0], [0.0, 0.0], [0.1, -0.3], [1.0, -1.0]])
    raw = torch.cat((_chol_raw_for(0.02, 0.0, 0.02), _chol_raw_for(0.02, 0.0, 0.02),
                     _chol_raw_for(50.0, 0.0, 50.0), _chol_raw_for(1e-4, 0.0, 1e-4),
                     _chol_raw_for(0.05, 0.0, 0.6)))
    b = _bounds(mu, raw, M, N)
    assert b.num_tile_rows == 3 and b.num_tile_cols == 5
    rects = torch.stack((b.tile_r0, b.tile_r1, b.tile_c0, b.tile_c1), 1).tolist()
    assert rects[0] == [0, 0, 0, 0]            # corner (-1,-1), clamped at 0
    assert rects[1] == [2, 2, 4, 4]            # corner (1,1): ragged last tile row and column
    assert rects[2] == [0, 2, 0, 4]            # sigma >> matrix: every tile
    # sigma << pixel: the centre's tile only (centre 24.2 rows, 24.15 cols)
    assert rects[3] == [1, 1, 1, 1]
    # (1,-1) with column std 0.6: ceil(0 + 3 * 0.6 * 0.5 * 69) = 63 -> tile 3; rows stay in tile 2
    assert rects[4] == [2, 2, 0, 3]
    assert b.tiles_touched.tolist() == [(r1 - r0 + 1) * (c1 - c0 + 1) for r0, r1, c0, c1 in rects]


def test_tile_bounds_against_float64():
    """Random Gaussians: the fp32 boxes equal a float64 recomputation except where a box edge
    lies within rounding distance of an integer pixel."""
    p = wl.make_problem("t", 300, 500, 3000, math.log(6.0), 0.9, seed=4, with_grad=False)
    b = _bounds(p.mu, p.chol_raw, 300, 500)
    L = fo.activate_cholesky(p.chol_raw).to(torch.float64)
    cov = L @ L.transpose(-1, -2)
    ok = 0
    for axis, (M, lo_t, hi_t) in enumerate(((300, b.tile_r0, b.tile_r1), (500, b.tile_c0, b.tile_c1))):
        std = torch.sqrt(cov[:, axis, axis].clamp_min(1e-8))
        centre = (p.mu[:, axis].to(torch.float64) + 1.0) * 0.5 * (M - 1)
        half = 3.0 * std * 0.5 * max(M - 1, 1)
        lo = torch.floor(centre - half).clamp(0, M - 1).to(torch.int64) // 16
        hi = torch.ceil(centre + half).clamp(0, M - 1).to(torch.int64) // 16
        near = (((centre - half) - torch.round(centre - half)).abs() < 1e-3) | \
               (((centre + half) - torch.round(centre + half)).abs() < 1e-3)
        assert torch.equal(lo[~near], lo_t[~near]) and torch.equal(hi[~near], hi_t[~near])
        ok += int((~near).sum())
    assert ok > 5900


# ------------------------------------------------------------------------------ tile index


def _brute_force_index(b: fo.TileBounds):
    ids, counts = [], []
    K = int(b.tile_r0.numel())
    for tr in range(b.num_tile_rows):
        for tc in range(b.num_tile_cols):
            here = [g for g in range(K) if int(b.tile_r0[g]) <= tr <= int(b.tile_r1[g])
                    and int(b.tile_c0[g]) <= tc <= int(b.tile_c1[g])]
            ids += here
            counts.append(len(here))
    ptr = [0]
    for c in counts:
        ptr.append(ptr[-1] + c)
    return torch.tensor(ptr, dtype=torch.int64), torch.tensor(ids, dtype=torch.int64)


@pytest.mark.parametrize("M,N,to,ti,K,seed", [(45, 70, 16, 16, 40, 1), (64, 64, 16, 16, 64, 2),
                                              (37, 101, 8, 24, 50, 3), (20, 20, 1, 1, 6, 4),
                                              (33, 17, 32, 32, 9, 5)])
def test_build_tile_index_brute_force(M, N, to, ti, K, seed):
    p = wl.make_problem("t", M, N, K, math.log(3.0), 1.0, seed=seed, with_grad=False)
    b = _bounds(p.mu, p.chol_raw, M, N, to, ti)
    idx = fo.build_tile_index(b)
    ptr, ids = _brute_force_index(b)
    assert torch.equal(idx.tile_ptr, ptr)
    assert torch.equal(idx.gaussian_ids, ids)
    assert int(idx.tile_ptr[-1]) == int(b.tiles_touched.sum())
    assert torch.all(idx.tile_ptr[1:] >= idx.tile_ptr[:-1])


def test_build_tile_index_empty():
    b = _bounds(torch.zeros(0, 2), torch.zeros(0, 3), 40, 40)
    idx = fo.build_tile_index(b)
    assert idx.tile_ptr.tolist() == [0] * 10 and idx.gaussian_ids.numel() == 0
    d, tp, ids = fo.gaussian_field_forward(*wl.axes(40, 40), torch.zeros(0, 2), torch.zeros(0, 3),
                                           torch.zeros(0, 1), 16, 16, 3.0)
    assert torch.count_nonzero(d) == 0 and ids.numel() == 0


# ------------------------------------------------------------------------------ render


@pytest.mark.parametrize("normalize,clamp", [(False, 80.0), (True, 80.0), (False, None), (False, 3.0)])
def test_render_single_gaussian_closed_form(normalize, clamp):
    M, N = 90, 120
    rc, cc = wl.axes(M, N)
    mu = torch.tensor([[0.1, -0.2]])
    raw = _chol_raw_for(0.12, 0.05, 0.09)
    amp = torch.tensor([[0.7]])
    d, tp, ids = fo.gaussian_field_forward(rc, cc, mu, raw, amp, 16, 16, 3.0, normalize, clamp)
    d = d.reshape(M, N).to(torch.float64)
    want = _exact_field(rc, cc, mu, fo.activate_cholesky(raw), amp, normalize, clamp)[0]
    mask = _tile_mask(_bounds(mu, raw, M, N), 0, M, N, 16, 16)
    assert torch.count_nonzero(d[~mask]) == 0, "pixels outside the tile rectangle must stay 0"
    scale = float(want.abs().max())
    assert float((d[mask] - want[mask]).abs().max()) <= 2e-6 * scale


def test_render_linear_in_amp_and_superposition():
    p = wl.make_problem("t", 64, 80, 10, math.log(4.0), 0.5, seed=7, with_grad=False)
    rc, cc = p.row_coords, p.col_coords
    d, tp, ids = fo.gaussian_field_forward(rc, cc, p.mu, p.chol_raw, p.amp, 16, 16, 3.0)
    d2, _, _ = fo.gaussian_field_forward(rc, cc, p.mu, p.chol_raw, 2.0 * p.amp, 16, 16, 3.0)
    assert torch.equal(d2, 2.0 * d)  # power-of-two scale is exact
    zero, _, _ = fo.gaussian_field_forward(rc, cc, p.mu, p.chol_raw, torch.zeros_like(p.amp), 16, 16, 3.0)
    assert torch.count_nonzero(zero) == 0
    total = torch.zeros_like(d, dtype=torch.float64)
    for g in range(p.k):
        dg, _, _ = fo.gaussian_field_forward(rc, cc, p.mu[g:g + 1], p.chol_raw[g:g + 1],
                                             p.amp[g:g + 1], 16, 16, 3.0)
        total += dg.to(torch.float64)
    assert float((total - d.to(torch.float64)).abs().max()) <= 1e-6 * float(total.abs().max())


def test_tiled_within_truncation_bound_of_dense():
    """|dense - tiled| at a pixel <= sum over Gaussians whose rectangle misses the pixel's tile
    of |amp| e^{-4.5} (outside the 3-sigma box q > 9); a mis-binned Gaussian breaks this."""
    M, N = 72, 88
    p = wl.make_problem("t", M, N, 14, math.log(4.0), 0.6, seed=3, with_grad=False)
    rc, cc = p.row_coords, p.col_coords
    tiled, _, _ = fo.gaussian_field_forward(rc, cc, p.mu, p.chol_raw, p.amp, 16, 16, 3.0)
    dense = fo.dense_field(rc, cc, p.mu, p.chol_raw, p.amp).reshape(M, N).to(torch.float64)
    b = _bounds(p.mu, p.chol_raw, M, N)
    bound = torch.zeros(M, N, dtype=torch.float64)
    for g in range(p.k):
        bound += (~_tile_mask(b, g, M, N, 16, 16)).to(torch.float64) * abs(float(p.amp[g])) * E45 * 1.001
    err = (dense - tiled.reshape(M, N).to(torch.float64)).abs()
    assert torch.all(err <= bound + 1e-6 * float(dense.abs().max()))
    assert float(err.max()) > 0  # the truncation is real


# ------------------------------------------------------------------------------ backward


def _fixed_index_render(p, index, dtype, normalize=False, clamp=None):
    def fn(mu, raw, amp):
        chol = fo.activate_cholesky(raw)
        return fo.render_tiles(p.row_coords.to(dtype), p.col_coords.to(dtype), mu, chol, amp, index,
                               16, 16, normalize, clamp)
    return fn


@pytest.mark.parametrize("normalize", [False, True])
def test_backward_gradcheck_fp64(normalize):
    p = wl.make_problem("t", 40, 36, 4, math.log(5.0), 0.3, seed=9, with_grad=False)
    b = _bounds(p.mu, p.chol_raw, 40, 36)
    index = fo.build_tile_index(b)
    f64 = torch.float64
    args = (p.mu.to(f64).requires_grad_(), p.chol_raw.to(f64).requires_grad_(),
            p.amp.to(f64).requires_grad_())
    assert torch.autograd.gradcheck(_fixed_index_render(p, index, f64, normalize), args,
                                    eps=1e-6, atol=1e-7, rtol=1e-5)


def test_d_amp_and_isotropic_d_mu_closed_form():
    M, N = 64, 64
    rc, cc = wl.axes(M, N)
    mu = torch.tensor([[0.05, -0.1], [-0.4, 0.3]])
    raw = torch.cat((_chol_raw_for(0.11, 0.0, 0.11), _chol_raw_for(0.07, 0.0, 0.07)))
    amp = torch.tensor([[0.8], [-0.5]])
    grad = torch.randn(M * N, generator=torch.Generator().manual_seed(5))
    _, _, _, d_mu, d_raw, d_amp = fo.gaussian_field_fwd_bwd(rc, cc, mu, raw, amp, grad, 16, 16, 3.0)
    L = fo.activate_cholesky(raw)
    b = _bounds(mu, raw, M, N)
    g64 = grad.reshape(M, N).to(torch.float64)
    unit = _exact_field(rc, cc, mu, L, torch.ones(2, 1))  # clamp 80 is inactive inside the boxes
    dx = (rc.to(torch.float64).reshape(-1, 1) - mu[:, 0].to(torch.float64).reshape(-1, 1, 1))
    dy = (cc.to(torch.float64).reshape(1, -1) - mu[:, 1].to(torch.float64).reshape(-1, 1, 1))
    for g in range(2):
        m = _tile_mask(b, g, M, N, 16, 16).to(torch.float64)
        want_amp = float((g64 * unit[g] * m).sum())
        assert abs(float(d_amp[g, 0]) - want_amp) <= 1e-5 * abs(want_amp) + 1e-6
        s2 = float(L[g, 0, 0].double() ** 2)  # isotropic: cov = l^2 I
        common = g64 * float(amp[g, 0]) * unit[g] * m / s2
        want_mu = torch.tensor([float((common * dx[g]).sum()), float((common * dy[g]).sum())])
        got = d_mu[g].to(torch.float64)
        assert float((got - want_mu).abs().max()) <= 1e-4 * float(want_mu.abs().max())


def test_covariance_chain_closed_form():
    """d(loss)/d(chol_raw) through cov = L L^T and softplus equals the textbook chain
    dl11 = 2 l11 G00 + l21 (G01 + G10), dl21 = l11 (G01 + G10) + 2 l21 G11, dl22 = 2 l22 G11,
    scaled by softplus' = sigmoid on the diagonal entries (backward.cu:436-496)."""
    g = torch.Generator().manual_seed(2)
    raw = (torch.randn(50, 3, generator=g, dtype=torch.float64) * 2.0).requires_grad_()
    G = torch.randn(50, 2, 2, generator=g, dtype=torch.float64)
    L = fo.activate_cholesky(raw)
    cov = L @ L.transpose(-1, -2)
    (d_raw,) = torch.autograd.grad((cov * G).sum(), raw)
    Ld = L.detach()
    l11, l21, l22 = Ld[:, 0, 0], Ld[:, 1, 0], Ld[:, 1, 1]
    off = G[:, 0, 1] + G[:, 1, 0]
    want = torch.stack((
        (2 * l11 * G[:, 0, 0] + l21 * off) * torch.sigmoid(raw[:, 0].detach()),
        l11 * off + 2 * l21 * G[:, 1, 1],
        2 * l22 * G[:, 1, 1] * torch.sigmoid(raw[:, 2].detach())), 1)
    assert torch.allclose(d_raw, want, rtol=1e-12, atol=1e-12)


def test_inverse_and_det_derivatives():
    """d(S^-1) = -S^-1 dS S^-1 and d det = det tr(S^-1 dS), by central differences."""
    g = torch.Generator().manual_seed(8)
    A = torch.randn(20, 2, 2, generator=g, dtype=torch.float64)
    S = A @ A.transpose(-1, -2) + 0.5 * torch.eye(2, dtype=torch.float64)
    dS = torch.randn(20, 2, 2, generator=g, dtype=torch.float64)
    dS = dS + dS.transpose(-1, -2)
    h = 1e-6
    inv_p, det_p = fo._inv_det(S + h * dS, False)
    inv_m, det_m = fo._inv_det(S - h * dS, False)
    Si = torch.linalg.inv(S)
    assert torch.allclose((inv_p - inv_m) / (2 * h), -Si @ dS @ Si, rtol=1e-6, atol=1e-7)
    tr = torch.einsum("kij,kji->k", Si, dS)
    assert torch.allclose((det_p - det_m) / (2 * h), torch.linalg.det(S) * tr, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------------------ variants


def _close(a, b, rtol):
    a, b = a.to(torch.float64), b.to(torch.float64)
    return float((a - b).abs().max()) <= rtol * float(b.abs().max()) + 1e-30


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3"])
def test_batched_and_fp64_variants_match_loop(cfg):
    p = wl.CONFIGS[cfg](0)
    args = (p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, 16, 16, 3.0, False, 80.0)
    loop = fo.gaussian_field_fwd_bwd(*args)
    batched = fo.gaussian_field_fwd_bwd_batched(*args)
    f64 = fo.gaussian_field_fwd_bwd_fp64(*args)
    fp32_linalg = fo.gaussian_field_fwd_bwd(*args, exact_linalg=False)
    for other, ftol, gtol in ((batched, 1e-6, 1e-5), (f64, 1e-5, 1e-4), (fp32_linalg, 1e-5, 1e-4)):
        assert torch.equal(other[1], loop[1]) and torch.equal(other[2], loop[2])
        assert _close(other[0], loop[0], ftol)
        for a, b in zip(other[3:], loop[3:]):
            assert _close(a, b, gtol)


def test_gaussian_linear_oracle_chains_through_tanh():
    """gaussian_linear_fwd_bwd (mu = tanh(mu_raw), autograd back through the tanh) against the
    field oracle at tanh(mu_raw) with d/dx tanh = 1 - tanh^2 applied in float64; a substituted
    forward value (mu_values) changes the field but keeps the derivative at tanh(mu_raw)."""
    p = wl.make_problem("tanh_chain", 48, 72, 20, math.log(3.0), 0.4, 21)
    mu_raw = torch.atanh(p.mu.clamp(-0.999999, 0.999999)) + 0.05
    args = (p.row_coords, p.col_coords)
    tail = (p.chol_raw, p.amp, p.grad, 16, 16, 3.0, False, 80.0)
    got = fo.gaussian_linear_fwd_bwd(*args, mu_raw, *tail)
    mu = torch.tanh(mu_raw)
    ref = fo.gaussian_field_fwd_bwd(*args, mu, *tail)
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]) and torch.equal(got[2], ref[2])
    t = torch.tanh(mu_raw.double())

    def chained(d_mu, d_mu_raw):
        # autograd forms 1 - y^2 from the fp32 tanh y: an absolute error of about 2^-23 in the
        # factor, i.e. relative 1e-5 where |tanh| is near 1 (mu_raw up to 3 here)
        want = d_mu.double() * (1.0 - t * t)
        err = (d_mu_raw.double() - want).abs()
        return bool((err <= 1e-6 * want.abs() + 3e-7 * d_mu.double().abs()).all())

    assert chained(ref[3], got[3])
    assert torch.equal(got[4], ref[4]) and torch.equal(got[5], ref[5])
    shifted = mu + 1e-3
    sub = fo.gaussian_linear_fwd_bwd(*args, mu_raw, *tail, mu_values=shifted)
    ref2 = fo.gaussian_field_fwd_bwd(*args, shifted, *tail)
    assert torch.equal(sub[0], ref2[0])
    assert chained(ref2[3], sub[3])
    batched = fo.gaussian_linear_fwd_bwd(*args, mu_raw, *tail, batched=True)
    assert _close(batched[0], got[0], 1e-6) and _close(batched[3], got[3], 1e-5)


# ------------------------------------------------------------------------------ fixtures


def test_golden_tiny_ragged():
    d = np.load(GOLDEN / "tiny_ragged.npz")
    t = lambda k: torch.from_numpy(d[k].copy())  # noqa: E731
    out = fo.gaussian_field_fwd_bwd(t("row_coords"), t("col_coords"), t("mu"), t("chol_raw"),
                                    t("amp"), t("grad"), 16, 16, 3.0, False, 80.0)
    assert torch.equal(out[1], t("tile_ptr")) and torch.equal(out[2], t("gaussian_ids"))
    assert _close(out[0], t("delta"), 1e-6)
    for a, k in zip(out[3:], ("d_mu", "d_chol_raw", "d_amp")):
        assert _close(a, t(k), 1e-5), k


def test_golden_cfg1_and_workload_generator():
    d = np.load(GOLDEN / "cfg1_seed0.npz")
    p = wl.cfg1(0)  # the generator must reproduce the recorded inputs bit for bit
    for k in ("mu", "chol_raw", "amp"):
        assert np.array_equal(getattr(p, k).numpy(), d[k]), k
    out = fo.gaussian_field_fwd_bwd(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad,
                                    16, 16, 3.0, False, 80.0)
    assert np.array_equal(out[1].numpy(), d["tile_ptr"])
    assert np.array_equal(out[2].numpy(), d["gaussian_ids"].astype(np.int64))
    pos = torch.from_numpy(d["delta_positions"].astype(np.int64))
    assert _close(out[0][pos], torch.from_numpy(d["delta_values"]), 1e-6)
    d64 = out[0].to(torch.float64)
    assert abs(float(d64.sum()) - float(d["delta_sum"])) <= 1e-6 * float(d64.abs().sum())
    assert abs(float((d64 * d64).sum()) - float(d["delta_sumsq"])) <= 1e-5 * float(d["delta_sumsq"])
    for a, k in zip(out[3:], ("d_mu", "d_chol_raw", "d_amp")):
        assert _close(a, torch.from_numpy(d[k]), 1e-5), k
