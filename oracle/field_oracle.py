"""CPU oracle for the Gaussian-field delta-W renderer -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
this module, and only as the checker or the timed CPU baseline.  The product path
(``guass_amd``) never calls it.

It restates, with the same PyTorch CPU tensor operations in the same order, the reference's
CPU/torch path for this kernel (paths are under ``/root/reference/gaussian_peft``):

* ``activate_cholesky``      kernels/covariance.py:14-26   (softplus + eps, strided views)
* ``tile_bounds``            kernels/bounds.py:24-75       (fp32 3-sigma box -> tile range)
* ``build_tile_index``       kernels/tile_index.py:51-99   (argsort made *stable*, see below)
* ``render_tiles``           kernels/tile_accumulate.py:95-131 with
                             kernels/gaussian_core.py:30-52,55-82 and covariance.py:29-38
* ``gaussian_field_forward`` the (delta, tile_ptr, gaussian_ids_sorted) triple that
                             cuda_field/csrc/field_impl.cu:135-163 returns
* ``gaussian_field_fwd_bwd`` forward + torch autograd backward, the gradient definition the
                             reference's training backward (backward.cu:541-716) implements
* ``gaussian_linear_fwd_bwd`` the layer's use of it: mu = tanh(mu_raw), autograd through the tanh
                             (layers/gaussian_linear.py:153-154,162-220)

Deliberate difference: the reference sorts pair keys with ``torch.argsort`` (default
``stable=False``, tile_index.py:86), whose within-tile order is implementation-defined.  The
canonical order is (tile ascending, gaussian id ascending) -- what the reference's CUDA path
produces with a stable radix sort over gid-major emission (forward.cu:226-240) -- so the
oracle uses ``stable=True``.

Parity pins (tests/test_oracle.py): brute-force enumeration of tile rectangles on tiny
inputs, closed-form single-Gaussian renders, a float64 dense evaluation, fp64 gradcheck,
closed-form cov-chain derivatives, and committed golden fixtures.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

CHOLESKY_EPS = 1e-5  # covariance.py eps as GaussianLinear passes it (config/adapter.py:19)


# --------------------------------------------------------------------------- geometry


def activate_cholesky(chol_raw: Tensor, eps: float = CHOLESKY_EPS) -> Tensor:
    """Lower-triangular L[K,2,2] from chol_raw[K,3] (covariance.py:14-26).

    Softplus is applied to strided column views exactly as the reference does; PyTorch then
    takes its scalar CPU branch (glibc expf/log1pf), which the GPU restates bit-exactly.
    """
    if chol_raw.ndim != 2 or chol_raw.shape[-1] != 3:
        raise ValueError("chol_raw must have shape [K, 3]")
    chol = torch.zeros(chol_raw.shape[0], 2, 2, dtype=chol_raw.dtype)
    chol[:, 0, 0] = F.softplus(chol_raw[:, 0]) + eps
    chol[:, 1, 0] = chol_raw[:, 1]
    chol[:, 1, 1] = F.softplus(chol_raw[:, 2]) + eps
    return chol


@dataclass
class TileBounds:
    tile_r0: Tensor
    tile_r1: Tensor
    tile_c0: Tensor
    tile_c1: Tensor
    tiles_touched: Tensor
    num_tile_rows: int
    num_tile_cols: int


def tile_bounds(
    mu: Tensor,
    chol: Tensor,
    out_features: int,
    in_features: int,
    tile_out: int,
    tile_in: int,
    sigma_multiplier: float,
) -> TileBounds:
    """fp32 sigma-box of every Gaussian, clamped to the matrix, as tile ranges (bounds.py:24-75).

    Operation order matters for bit-exactness: (mu + 1) * 0.5 * (M - 1) and
    sigma * std * 0.5 * max(M - 1, 1), each a separately rounded fp32 tensor op.
    """
    if out_features <= 0 or in_features <= 0:
        raise ValueError("out_features and in_features must be positive")
    if tile_out <= 0 or tile_in <= 0:
        raise ValueError("tile_out and tile_in must be positive")
    if sigma_multiplier <= 0:
        raise ValueError("sigma_multiplier must be positive")
    c32 = chol.to(dtype=torch.float32)
    cov = c32 @ c32.transpose(-1, -2)
    std_r = torch.sqrt(torch.clamp(cov[:, 0, 0], min=1e-8))
    std_c = torch.sqrt(torch.clamp(cov[:, 1, 1], min=1e-8))
    m32 = mu.to(dtype=torch.float32)
    centre_r = (m32[:, 0] + 1.0) * 0.5 * (out_features - 1)
    centre_c = (m32[:, 1] + 1.0) * 0.5 * (in_features - 1)
    half_r = sigma_multiplier * std_r * 0.5 * max(out_features - 1, 1)
    half_c = sigma_multiplier * std_c * 0.5 * max(in_features - 1, 1)
    row_lo = torch.floor(centre_r - half_r).to(dtype=torch.int64).clamp_(0, out_features - 1)
    row_hi = torch.ceil(centre_r + half_r).to(dtype=torch.int64).clamp_(0, out_features - 1)
    col_lo = torch.floor(centre_c - half_c).to(dtype=torch.int64).clamp_(0, in_features - 1)
    col_hi = torch.ceil(centre_c + half_c).to(dtype=torch.int64).clamp_(0, in_features - 1)
    n_tr = (out_features + tile_out - 1) // tile_out
    n_tc = (in_features + tile_in - 1) // tile_in
    tr0 = (row_lo // tile_out).clamp_(0, n_tr - 1)
    tr1 = (row_hi // tile_out).clamp_(0, n_tr - 1)
    tc0 = (col_lo // tile_in).clamp_(0, n_tc - 1)
    tc1 = (col_hi // tile_in).clamp_(0, n_tc - 1)
    touched = (tr1 - tr0 + 1) * (tc1 - tc0 + 1)
    return TileBounds(tr0, tr1, tc0, tc1, touched, n_tr, n_tc)


@dataclass
class TileIndex:
    tile_ptr: Tensor  # int64 [T+1]
    gaussian_ids: Tensor  # int64 [P], tile-major, gid ascending within a tile
    tile_ids: Tensor  # int64 [P]
    num_tile_rows: int
    num_tile_cols: int


def build_tile_index(b: TileBounds) -> TileIndex:
    """(tile, gaussian) pairs in canonical order and per-tile ranges (tile_index.py:51-99)."""
    k = int(b.tile_r0.shape[0])
    n_tiles = b.num_tile_rows * b.num_tile_cols
    total = int(b.tiles_touched.sum().item())
    if total == 0:
        empty = torch.empty(0, dtype=torch.int64)
        return TileIndex(torch.zeros(n_tiles + 1, dtype=torch.int64), empty, empty,
                         b.num_tile_rows, b.num_tile_cols)
    gid = torch.repeat_interleave(torch.arange(k, dtype=torch.int64), b.tiles_touched)
    first = torch.repeat_interleave(torch.cumsum(b.tiles_touched, 0) - b.tiles_touched, b.tiles_touched)
    local = torch.arange(total, dtype=torch.int64) - first
    width = (b.tile_c1 - b.tile_c0 + 1).index_select(0, gid)
    trow = b.tile_r0.index_select(0, gid) + torch.div(local, width, rounding_mode="floor")
    tcol = b.tile_c0.index_select(0, gid) + torch.remainder(local, width)
    tile = trow * b.num_tile_cols + tcol
    order = torch.argsort(tile, stable=True)
    tile = tile[order]
    gid = gid[order]
    counts = torch.bincount(tile, minlength=n_tiles)
    tile_ptr = torch.zeros(n_tiles + 1, dtype=torch.int64)
    tile_ptr[1:] = torch.cumsum(counts, 0)
    return TileIndex(tile_ptr, gid, tile, b.num_tile_rows, b.num_tile_cols)


# --------------------------------------------------------------------------- render


def _inv_det(cov: Tensor, exact_linalg: bool) -> tuple[Tensor, Tensor]:
    """torch.linalg.inv / det of the 2x2 covariances (gaussian_core.py:42-44, covariance.py:35-38).

    With ``exact_linalg`` the inverse and determinant of the same fp32 matrices are taken in
    float64 and rounded to fp32 (autograd runs through the casts).  fp32 LU carries an error of
    order cond(cov) * 2^-24 whose value depends on the BLAS (MKL) and the CPU; for the
    well-conditioned configs it is below fp32 rounding of the field, for strongly anisotropic
    Gaussians (cond up to 4e8 in cfg5) it is not, and only the exact form is reproducible.
    """
    if exact_linalg and cov.dtype == torch.float32:
        c64 = cov.to(torch.float64)
        return torch.linalg.inv(c64).to(cov.dtype), torch.linalg.det(c64).to(cov.dtype)
    return torch.linalg.inv(cov), torch.linalg.det(cov)


def _basis(coords: Tensor, mu: Tensor, inv_cov: Tensor, det_cov: Tensor, normalize: bool,
           clamp_quad: float | None) -> Tensor:
    """amp-free Gaussian basis [n, pixels] (gaussian_core.py:55-82)."""
    diff = coords.unsqueeze(0) - mu.unsqueeze(1)
    quad = torch.einsum("kmd,kde,kme->km", diff, inv_cov, diff)
    if clamp_quad is not None:
        quad = quad.clamp(min=0.0, max=clamp_quad)
    basis = torch.exp(-0.5 * quad)
    if normalize:
        norm = 1.0 / (2.0 * math.pi * torch.sqrt(det_cov).clamp_min(torch.finfo(coords.dtype).eps))
        basis = basis * norm.unsqueeze(-1)
    return basis


def render_tiles(row_coords: Tensor, col_coords: Tensor, mu: Tensor, chol: Tensor, amp: Tensor,
                 index: TileIndex, tile_out: int, tile_in: int, normalize: bool,
                 clamp_quad: float | None, exact_linalg: bool = True) -> Tensor:
    """Per-tile Python loop of the reference CPU path (tile_accumulate.py:95-131).

    Differentiable in mu, chol and amp.  Tiles are written by assignment; empty tiles stay 0.
    """
    m = int(row_coords.shape[0])
    n = int(col_coords.shape[0])
    dtype = row_coords.dtype
    inv_cov, det_cov = _inv_det(chol @ chol.transpose(-1, -2), exact_linalg)
    delta = torch.zeros(m, n, dtype=dtype)
    n_tc = index.num_tile_cols
    ptr = index.tile_ptr.tolist()
    for t in range(index.num_tile_rows * n_tc):
        s, e = ptr[t], ptr[t + 1]
        if s >= e:
            continue
        r0 = (t // n_tc) * tile_out
        c0 = (t % n_tc) * tile_in
        r1 = min(r0 + tile_out, m)
        c1 = min(c0 + tile_in, n)
        gr, gc = torch.meshgrid(row_coords[r0:r1], col_coords[c0:c1], indexing="ij")
        coords = torch.stack((gr, gc), dim=-1).reshape(-1, 2)
        ids = index.gaussian_ids[s:e]
        basis = _basis(coords, mu.index_select(0, ids), inv_cov.index_select(0, ids),
                       det_cov.index_select(0, ids), normalize, clamp_quad)
        tile_val = (amp.index_select(0, ids).reshape(-1, 1) * basis).sum(dim=0)
        delta[r0:r1, c0:c1] = tile_val.reshape(r1 - r0, c1 - c0).to(dtype=dtype)
    return delta.reshape(-1)


# --------------------------------------------------------------------------- entry points


def gaussian_field_forward(row_coords: Tensor, col_coords: Tensor, mu: Tensor, chol_raw: Tensor,
                           amp: Tensor, tile_out: int, tile_in: int, sigma_multiplier: float,
                           normalize: bool = False, clamp_quad: float | None = 80.0,
                           exact_linalg: bool = True):
    """(delta[M*N], tile_ptr[T+1] int64, gaussian_ids_sorted[P] int64), all CPU tensors."""
    chol = activate_cholesky(chol_raw)
    b = tile_bounds(mu, chol, int(row_coords.shape[0]), int(col_coords.shape[0]), tile_out,
                    tile_in, sigma_multiplier)
    index = build_tile_index(b)
    with torch.no_grad():
        delta = render_tiles(row_coords, col_coords, mu, chol, amp, index, tile_out, tile_in,
                             normalize, clamp_quad, exact_linalg)
    return delta, index.tile_ptr, index.gaussian_ids


def gaussian_field_fwd_bwd(row_coords: Tensor, col_coords: Tensor, mu: Tensor, chol_raw: Tensor,
                           amp: Tensor, grad_delta: Tensor, tile_out: int, tile_in: int,
                           sigma_multiplier: float, normalize: bool = False,
                           clamp_quad: float | None = 80.0, exact_linalg: bool = True):
    """Forward plus autograd backward through the same tensor program.

    Returns (delta, tile_ptr, gaussian_ids_sorted, d_mu[K,2], d_chol_raw[K,3], d_amp[K,1]).
    """
    mu_ = mu.detach().clone().requires_grad_(True)
    raw_ = chol_raw.detach().clone().requires_grad_(True)
    amp_ = amp.detach().clone().requires_grad_(True)
    chol = activate_cholesky(raw_)
    b = tile_bounds(mu_.detach(), chol.detach(), int(row_coords.shape[0]), int(col_coords.shape[0]),
                    tile_out, tile_in, sigma_multiplier)
    index = build_tile_index(b)
    delta = render_tiles(row_coords, col_coords, mu_, chol, amp_, index, tile_out, tile_in,
                         normalize, clamp_quad, exact_linalg)
    if delta.requires_grad:
        d_mu, d_raw, d_amp = torch.autograd.grad(delta, (mu_, raw_, amp_),
                                                 grad_outputs=grad_delta.reshape(-1).to(delta.dtype),
                                                 allow_unused=True)
    else:
        d_mu = d_raw = d_amp = None
    d_mu = torch.zeros_like(mu_) if d_mu is None else d_mu
    d_raw = torch.zeros_like(raw_) if d_raw is None else d_raw
    d_amp = torch.zeros_like(amp_) if d_amp is None else d_amp
    return delta.detach(), index.tile_ptr, index.gaussian_ids, d_mu, d_raw, d_amp


def gaussian_field_fwd_bwd_batched(row_coords: Tensor, col_coords: Tensor, mu: Tensor,
                                   chol_raw: Tensor, amp: Tensor, grad_delta: Tensor, tile_out: int,
                                   tile_in: int, sigma_multiplier: float, normalize: bool = False,
                                   clamp_quad: float | None = 80.0, pair_chunk: int = 65536,
                                   exact_linalg: bool = True):
    """Same tensor program as ``gaussian_field_fwd_bwd`` evaluated for all (tile, gaussian) pairs
    at once instead of a Python loop over tiles; only the fp32 summation order differs.  Used for
    full-size configurations where the loop's autograd graph is too slow.  Cross-checked against
    the loop form in tests/test_oracle.py.
    """
    mu_ = mu.detach().clone().requires_grad_(True)
    raw_ = chol_raw.detach().clone().requires_grad_(True)
    amp_ = amp.detach().clone().requires_grad_(True)
    m, n = int(row_coords.shape[0]), int(col_coords.shape[0])
    chol = activate_cholesky(raw_)
    b = tile_bounds(mu_.detach(), chol.detach(), m, n, tile_out, tile_in, sigma_multiplier)
    index = build_tile_index(b)
    inv_cov, det_cov = _inv_det(chol @ chol.transpose(-1, -2), exact_linalg)
    n_tc = index.num_tile_cols
    # padded pixel grid of every tile; out-of-matrix pixels are masked
    lr = torch.arange(tile_out)
    lc = torch.arange(tile_in)
    grad_flat = grad_delta.reshape(-1).to(row_coords.dtype)
    delta = torch.zeros(m * n, dtype=row_coords.dtype)
    loss = torch.zeros((), dtype=row_coords.dtype)
    P = int(index.gaussian_ids.numel())
    for s in range(0, P, pair_chunk):
        e = min(P, s + pair_chunk)
        tiles = index.tile_ids[s:e]
        ids = index.gaussian_ids[s:e]
        rows = (tiles // n_tc).unsqueeze(1) * tile_out + lr.unsqueeze(0)  # [p, to]
        cols = (tiles % n_tc).unsqueeze(1) * tile_in + lc.unsqueeze(0)    # [p, ti]
        rv = rows < m
        cv = cols < n
        rr = rows.clamp(max=m - 1)
        cc = cols.clamp(max=n - 1)
        gr = row_coords[rr].unsqueeze(2).expand(-1, -1, tile_in)
        gc = col_coords[cc].unsqueeze(1).expand(-1, tile_out, -1)
        coords = torch.stack((gr, gc), dim=-1).reshape(e - s, -1, 2)          # [p, px, 2]
        valid = (rv.unsqueeze(2) & cv.unsqueeze(1)).reshape(e - s, -1)
        flat = (rr.unsqueeze(2) * n + cc.unsqueeze(1)).reshape(e - s, -1)
        diff = coords - mu_.index_select(0, ids).unsqueeze(1)
        quad = torch.einsum("kmd,kde,kme->km", diff, inv_cov.index_select(0, ids), diff)
        if clamp_quad is not None:
            quad = quad.clamp(min=0.0, max=clamp_quad)
        basis = torch.exp(-0.5 * quad)
        if normalize:
            nrm = 1.0 / (2.0 * math.pi * torch.sqrt(det_cov.index_select(0, ids))
                         .clamp_min(torch.finfo(row_coords.dtype).eps))
            basis = basis * nrm.unsqueeze(-1)
        contrib = amp_.index_select(0, ids).reshape(-1, 1) * basis * valid
        delta.index_add_(0, flat[valid], contrib.detach()[valid])
        loss = loss + (contrib * grad_flat[flat]).sum()
    if loss.requires_grad:
        d_mu, d_raw, d_amp = torch.autograd.grad(loss, (mu_, raw_, amp_), allow_unused=True)
    else:
        d_mu = d_raw = d_amp = None
    d_mu = torch.zeros_like(mu_) if d_mu is None else d_mu
    d_raw = torch.zeros_like(raw_) if d_raw is None else d_raw
    d_amp = torch.zeros_like(amp_) if d_amp is None else d_amp
    return delta, index.tile_ptr, index.gaussian_ids, d_mu, d_raw, d_amp


def gaussian_field_fwd_bwd_fp64(row_coords: Tensor, col_coords: Tensor, mu: Tensor,
                                chol_raw: Tensor, amp: Tensor, grad_delta: Tensor, tile_out: int,
                                tile_in: int, sigma_multiplier: float, normalize: bool = False,
                                clamp_quad: float | None = 80.0):
    """The batched program evaluated in float64 on the same fp32 inputs, with the binning, the
    activated Cholesky factor and the covariance computed in fp32 exactly as the reference does
    (so the same Gaussians and the same pairs), then every later step in float64.  Accuracy
    yardstick for ill-conditioned Gaussians, where no two fp32 evaluation orders agree.
    """
    chol32 = activate_cholesky(chol_raw)
    cov32 = chol32 @ chol32.transpose(-1, -2)
    b = tile_bounds(mu, chol32, int(row_coords.shape[0]), int(col_coords.shape[0]), tile_out, tile_in,
                    sigma_multiplier)
    index = build_tile_index(b)
    f64 = torch.float64
    mu_ = mu.to(f64).requires_grad_(True)
    raw_ = chol_raw.to(f64).requires_grad_(True)
    amp_ = amp.to(f64).requires_grad_(True)
    # L from fp64 softplus, with the fp32 values substituted (straight-through) so that the
    # covariance is the reference's fp32 one while gradients flow in float64.
    chol64 = torch.zeros(raw_.shape[0], 2, 2, dtype=f64)
    sp11 = F.softplus(raw_[:, 0]) + CHOLESKY_EPS
    sp22 = F.softplus(raw_[:, 2]) + CHOLESKY_EPS
    chol64[:, 0, 0] = sp11 + (chol32[:, 0, 0].to(f64) - sp11).detach()
    chol64[:, 1, 0] = raw_[:, 1]
    chol64[:, 1, 1] = sp22 + (chol32[:, 1, 1].to(f64) - sp22).detach()
    cov64 = chol64 @ chol64.transpose(-1, -2)
    cov64 = cov64 + (cov32.to(f64) - cov64).detach()
    inv_cov = torch.linalg.inv(cov64)
    det_cov = torch.linalg.det(cov64)
    m, n = int(row_coords.shape[0]), int(col_coords.shape[0])
    rc, cc = row_coords.to(f64), col_coords.to(f64)
    grad_flat = grad_delta.reshape(-1).to(f64)
    delta = torch.zeros(m * n, dtype=f64)
    loss = torch.zeros((), dtype=f64)
    n_tc = index.num_tile_cols
    lr, lc = torch.arange(tile_out), torch.arange(tile_in)
    P = int(index.gaussian_ids.numel())
    for s in range(0, P, 32768):
        e = min(P, s + 32768)
        tiles, ids = index.tile_ids[s:e], index.gaussian_ids[s:e]
        rows = (tiles // n_tc).unsqueeze(1) * tile_out + lr.unsqueeze(0)
        cols = (tiles % n_tc).unsqueeze(1) * tile_in + lc.unsqueeze(0)
        valid = ((rows < m).unsqueeze(2) & (cols < n).unsqueeze(1)).reshape(e - s, -1)
        rr, cl = rows.clamp(max=m - 1), cols.clamp(max=n - 1)
        dx = (rc[rr].unsqueeze(2) - mu_[ids, 0].view(-1, 1, 1)).expand(-1, -1, tile_in)
        dy = (cc[cl].unsqueeze(1) - mu_[ids, 1].view(-1, 1, 1)).expand(-1, tile_out, -1)
        A = inv_cov.index_select(0, ids)
        quad = (A[:, 0, 0].view(-1, 1, 1) * dx * dx + (A[:, 0, 1] + A[:, 1, 0]).view(-1, 1, 1) * dx * dy
                + A[:, 1, 1].view(-1, 1, 1) * dy * dy).reshape(e - s, -1)
        if clamp_quad is not None:
            quad = quad.clamp(min=0.0, max=clamp_quad)
        basis = torch.exp(-0.5 * quad)
        if normalize:
            nrm = 1.0 / (2.0 * math.pi * torch.sqrt(det_cov.index_select(0, ids))
                         .clamp_min(torch.finfo(torch.float32).eps))
            basis = basis * nrm.unsqueeze(-1)
        contrib = amp_.index_select(0, ids).reshape(-1, 1) * basis * valid
        flat = (rr.unsqueeze(2) * n + cl.unsqueeze(1)).reshape(e - s, -1)
        delta.index_add_(0, flat[valid], contrib.detach()[valid])
        loss = loss + (contrib * grad_flat[flat]).sum()
    d_mu, d_raw, d_amp = torch.autograd.grad(loss, (mu_, raw_, amp_), allow_unused=True)
    z = lambda g, like: torch.zeros_like(like) if g is None else g  # noqa: E731
    return delta, index.tile_ptr, index.gaussian_ids, z(d_mu, mu_), z(d_raw, raw_), z(d_amp, amp_)


def dense_field(row_coords: Tensor, col_coords: Tensor, mu: Tensor, chol_raw: Tensor, amp: Tensor,
                normalize: bool = False, clamp_quad: float | None = 80.0) -> Tensor:
    """Untruncated sum over all K Gaussians at every pixel (kernels/gaussian_field.py:100-127).

    Memory is K*M*N; tiny inputs only.  Differs from the tiled field by the tails cut at the
    sigma box, so it is a cross-check for Gaussians well inside their boxes.
    """
    chol = activate_cholesky(chol_raw)
    gr, gc = torch.meshgrid(row_coords, col_coords, indexing="ij")
    coords = torch.stack((gr, gc), dim=-1).reshape(-1, 2)
    inv_cov, det_cov = _inv_det(chol @ chol.transpose(-1, -2), True)
    basis = _basis(coords, mu, inv_cov, det_cov, normalize, clamp_quad)
    return (amp.reshape(-1, 1) * basis).sum(dim=0)



def gaussian_linear_fwd_bwd(row_coords: Tensor, col_coords: Tensor, mu_raw: Tensor, chol_raw: Tensor,
                            amp: Tensor, grad_delta: Tensor, tile_out: int, tile_in: int,
                            sigma_multiplier: float, normalize: bool = False,
                            clamp_quad: float | None = 80.0, *, mu_values: Tensor | None = None,
                            batched: bool = False, exact_linalg: bool = True):
    """The field of ``GaussianLinear.compute_delta_weight`` (layers/gaussian_linear.py:153-154,
    162-220): mu = tanh(mu_raw), the field program on it, and autograd back through the tanh.

    ``mu_values`` (optional, fp32 [K,2]) substitutes the forward value of tanh(mu_raw) -- e.g. the
    device's tanh, which may differ from the CPU's in the last ulp and so move a sigma box across
    a tile edge -- while the gradient still flows through ``torch.tanh``'s autograd.
    Returns (delta, tile_ptr, gaussian_ids_sorted, d_mu_raw[K,2], d_chol_raw[K,3], d_amp[K,1]).
    """
    raw_leaf = mu_raw.detach().clone().requires_grad_(True)
    mu = torch.tanh(raw_leaf)
    if mu_values is not None:
        mu = mu + (mu_values.to(mu.dtype) - mu).detach()
    fn = gaussian_field_fwd_bwd_batched if batched else gaussian_field_fwd_bwd
    out = fn(row_coords, col_coords, mu.detach(), chol_raw, amp, grad_delta, tile_out, tile_in,
             sigma_multiplier, normalize, clamp_quad, exact_linalg=exact_linalg)
    (d_mu_raw,) = torch.autograd.grad(mu, raw_leaf, grad_outputs=out[3])
    return out[0], out[1], out[2], d_mu_raw, out[4], out[5]
