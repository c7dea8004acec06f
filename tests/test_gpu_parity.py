"""GPU parity of libgaussfield.so against the CPU oracle (runs on an MI355X).

Every test calls the product path (guass_amd.cuda_field.ext -> C ABI -> gfx950 kernels) and
compares with oracle/field_oracle.py on the same seeded fp32 inputs, at the bars of
tests/parity.py.
"""

from __future__ import annotations

import ctypes
import math
import warnings

import pytest
import torch

from guass_amd import _native
from guass_amd import workloads as wl
from guass_amd.cuda_field import ext, runtime
from guass_amd.ops import FieldPlan
from oracle import field_oracle as fo
from tests.parity import HEAVY_TILE, SOFTPLUS_CHECKSUM, binning_equal, field_close, grad_close

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(f"[gpu-test] {msg}", flush=True)


def run_gpu(p: wl.FieldProblem, device, tile_out=16, tile_in=16, sigma=3.0, normalize=False,
            clamp=80.0, index_dtype=torch.int64):
    q = p.to(device)
    delta, tp, ids = ext.gaussian_field_forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                tile_out, tile_in, sigma, normalize, clamp)
    d_mu, d_raw, d_amp = ext.gaussian_field_backward(
        q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, tp.to(index_dtype),
        ids.to(index_dtype), tile_out, tile_in, sigma, normalize, clamp)
    torch.cuda.synchronize()
    return delta, tp, ids, d_mu, d_raw, d_amp


def oracle(p: wl.FieldProblem, tile_out=16, tile_in=16, sigma=3.0, normalize=False, clamp=80.0,
           batched=False, exact_linalg=True):
    fn = fo.gaussian_field_fwd_bwd_batched if batched else fo.gaussian_field_fwd_bwd
    return fn(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, tile_out, tile_in, sigma,
              normalize, clamp, exact_linalg=exact_linalg)


def check(p: wl.FieldProblem, device, batched=False, exact_linalg=True, **kw):
    say(f"{p.name} M={p.out_features} N={p.in_features} K={p.k} {kw}"
        + ("" if exact_linalg else " (oracle: fp32 linalg.inv/det)"))
    g = run_gpu(p, device, **kw)
    r = oracle(p, batched=batched, exact_linalg=exact_linalg, **kw)
    binning_equal(g[1], g[2], r[1], r[2])
    errs = {"delta": field_close(g[0], r[0])}
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), g[3:], r[3:]):
        errs[name] = grad_close(a, b, name)
    say(f"  ok pairs={int(r[1][-1])} " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    return g, r


def accuracy_check(p: wl.FieldProblem, device, tile_out=16, tile_in=16, sigma=3.0, normalize=False, clamp=80.0):
    """Binning bit-exact; delta-W and gradients at least as close to the float64 evaluation of
    the reference program as the fp32 oracle is (for ill-conditioned covariances)."""
    kw = dict(tile_out=tile_out, tile_in=tile_in, sigma=sigma, normalize=normalize, clamp=clamp)
    say(f"{p.name} M={p.out_features} N={p.in_features} K={p.k} {kw} (vs float64)")
    g = run_gpu(p, device, **kw)
    o = oracle(p, batched=True, **kw)
    r = fo.gaussian_field_fwd_bwd_fp64(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad,
                                       tile_out, tile_in, sigma, normalize, clamp)
    binning_equal(g[1], g[2], r[1], r[2])
    binning_equal(o[1], o[2], r[1], r[2])
    if p.k == 0:
        assert float(g[0].abs().max()) == 0.0
        return
    finite = torch.isfinite(r[0])
    assert torch.equal(torch.isfinite(g[0].cpu()), finite), "non-finite values differ from float64"
    scale = max(float(r[0][finite].abs().max()) if finite.any() else 0.0, 1e-30)
    err_g = float((g[0].cpu().double() - r[0])[finite].abs().max()) / scale if finite.any() else 0.0
    err_o = float((o[0].double() - r[0])[finite].abs().max()) / scale if finite.any() else 0.0
    say(f"  delta vs fp64: gpu {err_g:.2e} oracle {err_o:.2e}")
    assert err_g <= err_o + 1e-5
    # Per Gaussian, the gradient row (d_mu, d_chol_raw, d_amp) is finite exactly where float64's
    # is. Within a non-finite row the split between NaN and 0 in d_mu depends on which pixels a
    # numerically singular covariance clamps, which fp32 rounding decides (the fp32 oracle and
    # float64 disagree there too).
    def rows_finite(grads):
        return torch.stack([torch.isfinite(t.cpu().reshape(p.k, -1)).all(-1) for t in grads]).all(0)

    fin_rows = rows_finite(r[3:])
    assert torch.equal(rows_finite(g[3:]), fin_rows), "non-finite gradient rows differ from float64"
    assert torch.equal(rows_finite(o[3:]), fin_rows), "oracle: non-finite gradient rows differ"
    for name, a, b, c in zip(("d_mu", "d_chol_raw", "d_amp"), g[3:], o[3:], r[3:]):
        a, b = a.cpu().double()[fin_rows], b.double()[fin_rows]
        c = c[fin_rows]
        fin = torch.isfinite(c)
        assert torch.equal(torch.isfinite(a), fin), f"{name}: non-finite values differ from float64"
        cn = float(c[fin].norm())
        if cn == 0.0:
            continue
        eg = float((a - c)[fin].norm()) / cn
        eo = float((b - c)[fin].norm()) / cn
        say(f"  {name} vs fp64: gpu {eg:.2e} oracle {eo:.2e}")
        assert eg <= eo + 1e-4, name


def tiny_problem(M, N, K, seed, log_scale_px=1.5, spread=0.4):
    return wl.make_problem(f"tiny_{M}x{N}_k{K}_s{seed}", M, N, K, log_scale_px, spread, seed)


# ------------------------------------------------------------------------------------------

def test_softplus_selftest_matches_host_libm(device):
    say("softplus self-test over 2^32 inputs")
    h = ctypes_u64()
    _native.check(_native.lib().gf_selftest_softplus(h, None), "gf_selftest_softplus")
    assert h.value == SOFTPLUS_CHECKSUM, hex(h.value)


def ctypes_u64():
    import ctypes

    return ctypes.c_uint64(0)


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3"])
def test_parity_baseline_configs(cfg, device):
    check(wl.CONFIGS[cfg](0), device)


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3"])
def test_parity_reference_fp32_linalg(cfg, device):
    """The same configs against the oracle with the reference CPU path's literal fp32
    torch.linalg.inv / det (kernels/covariance.py:35-38, gaussian_core.py:42-44) instead of the
    exact inverse of the same fp32 covariance: the kernels meet the bars against both."""
    check(wl.CONFIGS[cfg](0), device, exact_linalg=False)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_parity_cfg2_more_seeds(seed, device):
    check(wl.cfg2(seed), device)


def test_parity_cfg5c_full_size(device):
    # cfg5 size, clustering and load imbalance, log-scales clipped (condition number <= 403)
    check(wl.cfg5c(0), device, batched=True)


@pytest.mark.parametrize("t_scale", [0.5, 1.0])
def test_accuracy_cfg5_full_size(device, t_scale):
    """cfg5 proper: Student-t log-scales give covariances with condition numbers up to 4e8,
    for which no two fp32 evaluation orders of the field agree to 1e-5 (the reference's own fp32
    path is 1.3e-2 away from a float64 evaluation of the same program).  Binning must still be
    bit-exact; field and gradients must be at least as close to the float64 evaluation as the
    CPU oracle (reference program with exact 2x2 linear algebra) is.  t_scale 1.0 is the stress
    variant (1.67M pairs, dense tiles of up to 255 Gaussians), whose widest scales overflow the
    generator's log(expm1(.)) to chol_raw = inf for four Gaussians: the reference program then
    gives non-finite delta-W on their tiles and non-finite gradients for them, and the GPU must
    give non-finite values at exactly those places, the finite ones compared as above."""
    p = wl.cfg5(0, t_scale=t_scale)
    say(f"{p.name} accuracy vs float64")
    g = run_gpu(p, device)
    o = oracle(p, batched=True)
    r = fo.gaussian_field_fwd_bwd_fp64(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad,
                                       16, 16, 3.0)
    binning_equal(g[1], g[2], r[1], r[2])
    binning_equal(o[1], o[2], r[1], r[2])
    fin = torch.isfinite(r[0])
    assert torch.equal(torch.isfinite(g[0].cpu()), fin) and torch.equal(torch.isfinite(o[0]), fin)
    scale = float(r[0][fin].abs().max())
    err_g = float((g[0].cpu().double() - r[0])[fin].abs().max()) / scale
    err_o = float((o[0].double() - r[0])[fin].abs().max()) / scale
    say(f"  delta vs fp64: gpu {err_g:.2e} oracle {err_o:.2e} ({int((~fin).sum())} non-finite)")
    assert err_g <= err_o + 1e-5
    for name, a, b, c in zip(("d_mu", "d_chol_raw", "d_amp"), g[3:], o[3:], r[3:]):
        fc = torch.isfinite(c)
        assert torch.equal(torch.isfinite(a.cpu()), fc), name
        eg = float((a.cpu().double() - c)[fc].norm() / c[fc].norm())
        eo = float((b.double() - c)[fc].norm() / c[fc].norm())
        say(f"  {name} vs fp64: gpu {eg:.2e} oracle {eo:.2e}")
        assert eg <= eo + 1e-4, name


def test_ragged_tiles(device):
    check(tiny_problem(37, 53, 20, 4), device)


def test_tiles_32x32(device):
    check(wl.cfg1(0), device, tile_out=32, tile_in=32)


@pytest.mark.parametrize("which", ["cfg3", "ragged", "cfg2"])
def test_tiles_32x32_quadrants(device, which):
    """32x32 tiles (the reference's training configs, configs/dreambooth_sd*.yaml:27-28): four
    16x16 quadrant waves per tile on the mask path."""
    p = {"cfg3": lambda: wl.cfg3(4), "ragged": lambda: tiny_problem(100, 90, 40, 14),
         "cfg2": lambda: wl.cfg2(6)}[which]()
    check(p, device, tile_out=32, tile_in=32)


def test_tiles_32x32_emission_path(device):
    # K > 8192: emission path; the render stays on the any-shape kernel, the backward on quadrants
    p = tiny_problem(96, 112, 9000, 15, log_scale_px=-1.0, spread=0.3)
    check(p, device, batched=True, tile_out=32, tile_in=32)


def test_batch_32x32_tiles(device):
    from guass_amd.ops import FieldBatchPlan

    probs = [wl.cfg1(3), wl.cfg2(4), tiny_problem(45, 70, 12, 12)]
    singles = [run_gpu(p, device, tile_out=32, tile_in=32) for p in probs]
    batch = FieldBatchPlan([p.to(device) for p in probs], device, capacities=[int(s[1][-1]) for s in singles],
                           tile_out=32, tile_in=32)
    batch.forward()
    batch.backward()
    torch.cuda.synchronize()
    assert batch.status() == [0] * len(probs)
    for i, (pl, sg) in enumerate(zip(batch.plans, singles)):
        P = int(sg[1][-1])
        assert torch.equal(pl.tile_ptr, sg[1]) and torch.equal(pl.ids[:P], sg[2]), f"layer {i}: binning"
        assert torch.equal(pl.delta, sg[0]), f"layer {i}: delta"
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), sg[3:]):
            grad_close(a, b, f"layer {i} {name}", rtol=1e-5)


def test_tiles_8x24(device):
    check(tiny_problem(100, 90, 40, 5), device, tile_out=8, tile_in=24)


def test_tiles_1x1(device):
    check(tiny_problem(24, 20, 6, 6, log_scale_px=0.7), device, tile_out=1, tile_in=1)


def test_normalize(device):
    check(wl.cfg1(0), device, normalize=True)


def test_no_clamp(device):
    check(wl.cfg2(0), device, clamp=None)


def test_sigma_multiplier_2_5(device):
    check(wl.cfg2(1), device, sigma=2.5)


@pytest.mark.parametrize("shape", [(100, 200), (1250, 700)])
@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("k", [1, 31, 32, 33, 63, 64, 65, 127, 129, 257, 1000, 2048, 2049, 8192])
def test_mask_path_binning_k_boundaries(device, k, tile, shape):
    """The mask path's binning at K around the 64-Gaussian ballot groups (a mask word pair each),
    around the preparation's lane split (four lanes per Gaussian up to 2048, one above) and at
    the path's largest K, with Gaussians spanning the whole grid and Gaussians in the
    last, partial tile row and column.  K <= 256 bins in the render, larger K in k_bin_tiles (a
    workgroup per tile row and column): tile_ptr and ids bit-exact against the oracle's binning
    (bounds.py:24-75, tile_index.py:51-99), delta-W at the field tolerance on the small grid."""
    M, N = shape
    p = tiny_problem(M, N, k, 40 + k, log_scale_px=1.5 if M < 1000 else 3.0, spread=0.9)
    g = torch.Generator().manual_seed(k)
    huge = torch.arange(0, k, 7)
    p.chol_raw[huge] = torch.tensor([3.0, 0.2, 3.0])  # sigma boxes past the matrix
    corner = torch.arange(k)[3::11]
    p.mu[corner] = torch.tensor([0.98, 0.99]) + 0.01 * torch.rand(len(corner), 2, generator=g)
    say(f"mask-path binning {M}x{N} K={k} tile {tile}")
    q = p.to(device)
    delta, tp, ids = ext.gaussian_field_forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                tile, tile, 3.0, False, 80.0)
    torch.cuda.synchronize()
    chol = fo.activate_cholesky(p.chol_raw)
    ti = fo.build_tile_index(fo.tile_bounds(p.mu, chol, p.out_features, p.in_features, tile, tile, 3.0))
    binning_equal(tp, ids, ti.tile_ptr, ti.gaussian_ids)
    if k <= 1000 and M < 1000:
        ref = fo.gaussian_field_forward(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, tile, tile,
                                        3.0, False, 80.0)[0]
        field_close(delta, ref)


@pytest.mark.parametrize("tile", [16, 32])
def test_dense_tiles_backward(device, tile):
    """Tiles of many Gaussians (P >= 16 T: the single-field backward takes the transposing
    moment reduction) against the oracle."""
    p = tiny_problem(256, 256, 2048, 21, log_scale_px=2.5)
    g, r = check(p, device, batched=True, tile_out=tile, tile_in=tile)
    assert int(r[1][-1]) >= 16 * (256 // tile) ** 2, "not dense enough for the transposing reduction"


def _random_cases(n: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    tiles = [(16, 16), (32, 32), (16, 16), (8, 24), (32, 16), (4, 4)]
    for i in range(n):
        M = int(torch.randint(1, 140, (1,), generator=g))
        N = int(torch.randint(1, 140, (1,), generator=g))
        K = int(torch.randint(0, 300, (1,), generator=g))
        to, ti = tiles[i % len(tiles)]
        log_scale = float(torch.empty(1).uniform_(0.0, 3.0, generator=g))
        sigma = float(torch.empty(1).uniform_(1.5, 3.5, generator=g))
        clamp = None if i % 5 == 4 else float(torch.empty(1).uniform_(20.0, 100.0, generator=g))
        yield i, M, N, K, to, ti, log_scale, sigma, clamp, i % 7 == 3


@pytest.mark.parametrize("case", list(_random_cases(40, 2026)), ids=lambda c: f"r{c[0]}")
def test_random_fields(device, case):
    """Seeded random fields over sizes (ragged and tiny), K (including 0), tile shapes (the
    mask path's 16x16 / 32x32, the emission path's others), sigma multiplier, clamp (or none)
    and normalisation: binning bit-exact, delta-W and gradients at the parity bars."""
    i, M, N, K, to, ti, log_scale, sigma, clamp, normalize = case
    p = wl.make_problem(f"rand{i}", M, N, K, log_scale, 0.6, 100 + i)
    check(p, device, tile_out=to, tile_in=ti, sigma=sigma, clamp=clamp, normalize=normalize)


@pytest.mark.parametrize("tile", [16, 32])
def test_low_clamp_backward(device, tile):
    """clamp_quad below 80: pixels with q > clamp carry no quadratic-form gradient (the
    reference's clamp mask, backward.cu:316-320,336-338), for the single-field backward (sparse
    and dense tiles) and the batched one, against the oracle."""
    from guass_amd.ops import FieldBatchPlan

    sparse = wl.make_problem("clamp_sparse", 320, 320, 200, math.log(5.0), 0.6, 31)
    dense = tiny_problem(128, 128, 800, 32, log_scale_px=2.5)
    for p in (sparse, dense):
        check(p, device, tile_out=tile, tile_in=tile, clamp=22.0)
    refs = [oracle(p, tile_out=tile, tile_in=tile, clamp=22.0) for p in (sparse, dense)]
    batch = FieldBatchPlan([p.to(device) for p in (sparse, dense)], device,
                           capacities=[int(r[1][-1]) for r in refs], tile_out=tile, tile_in=tile, clamp_quad=22.0)
    assert batch.info.mask_clamp == 1
    batch.forward()
    batch.backward()
    torch.cuda.synchronize()
    assert batch.status() == [0, 0]
    for i, (pl, r) in enumerate(zip(batch.plans, refs)):
        field_close(pl.delta, r[0])
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), r[3:]):
            grad_close(a, b, f"batch layer {i} {name}")


def _wide_cases(n: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    tiles = [(16, 16), (32, 32), (1, 7), (13, 5), (64, 64), (16, 16), (32, 32)]
    for i in range(n):
        M = int(torch.randint(1, 520, (1,), generator=g))
        N = int(torch.randint(1, 520, (1,), generator=g))
        K = int(torch.randint(8193, 8600, (1,), generator=g)) if i % 9 == 5 else int(torch.randint(0, 1500, (1,), generator=g))
        to, ti = tiles[i % len(tiles)]
        if to * ti < 64:  # keep the oracle's tile count small
            M, N = min(M, 96), min(N, 96)
        log_scale = float(torch.empty(1).uniform_(-1.0, 3.5, generator=g))
        sigma = float(torch.empty(1).uniform_(0.5, 4.0, generator=g))
        clamp = None if i % 6 == 1 else float(torch.empty(1).uniform_(1.0, 200.0, generator=g))
        shear = float(torch.empty(1).uniform_(0.0, 3.0, generator=g))
        yield i, M, N, K, to, ti, log_scale, sigma, clamp, i % 4 == 2, shear


@pytest.mark.parametrize("case", list(_wide_cases(30, 77)), ids=lambda c: f"w{c[0]}")
def test_random_fields_wide(device, case):
    """Wider seeded sweep: grids up to 519, K up to 1499 and past the mask path (8193..8599, the
    emission path at 16x16), tiles 1x7, 13x5, 64x64 besides 16x16 / 32x32, sub-pixel to large
    Gaussians, sheared (strongly anisotropic) covariances, clamp 1..200 or none, sigma 0.5..4,
    normalisation.  Sheared covariances are ill-conditioned, where no two fp32 evaluation orders
    agree to 1e-5, so the yardstick is the float64 evaluation of the same program: binning
    bit-exact, field and gradients at least as close to it as the fp32 oracle."""
    i, M, N, K, to, ti, log_scale, sigma, clamp, normalize, shear = case
    p = wl.make_problem(f"wide{i}", M, N, K, log_scale, 0.8, 300 + i)
    if K:
        gen = torch.Generator().manual_seed(400 + i)
        p.chol_raw[:, 1] += shear * torch.randn(K, generator=gen)
    accuracy_check(p, device, tile_out=to, tile_in=ti, sigma=sigma, clamp=clamp, normalize=normalize)


def test_k1_corner_and_huge(device):
    # one Gaussian at the top-left corner, one covering the whole matrix
    p = tiny_problem(70, 90, 2, 7)
    p.mu[0] = torch.tensor([-1.0, -1.0])
    p.mu[1] = torch.tensor([0.1, -0.2])
    p.chol_raw[1] = torch.tensor([2.0, 0.5, 1.5])
    check(p, device)


def test_tiny_sigma_single_tile(device):
    # sub-pixel Gaussians: one tile each unless the box straddles a tile border
    p = tiny_problem(64, 64, 30, 8, log_scale_px=-3.0, spread=0.1)
    g, r = check(p, device)
    assert p.k <= int(r[1][-1]) < 2 * p.k


def test_k_zero(device):
    p = tiny_problem(40, 33, 1, 9)
    p.mu, p.chol_raw, p.amp = p.mu[:0], p.chol_raw[:0], p.amp[:0]
    q = p.to(device)
    delta, tp, ids = ext.gaussian_field_forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                16, 16, 3.0, False, 80.0)
    d_mu, d_raw, d_amp = ext.gaussian_field_backward(q.grad, q.row_coords, q.col_coords, q.mu,
                                                     q.chol_raw, q.amp, tp, ids, 16, 16, 3.0, False, 80.0)
    torch.cuda.synchronize()
    assert delta.shape == (40 * 33,) and float(delta.abs().max()) == 0.0
    assert tp.shape == (3 * 3 + 1,) and int(tp.abs().max()) == 0 and ids.numel() == 0
    assert d_mu.shape == (0, 2) and d_raw.shape == (0, 3) and d_amp.shape == (0, 1)


def test_long_segments_bitmap_path(device):
    # ~3100 Gaussians per tile (> 2048 LDS keys, K <= 131072): bitmap ordering
    p = tiny_problem(64, 64, 50000, 10, log_scale_px=-3.0, spread=0.1)
    check(p, device, batched=True)


def test_long_segments_global_path(device):
    # K > 131072 with ~8800 Gaussians per tile: in-place global-memory ordering
    p = tiny_problem(64, 64, 140000, 11, log_scale_px=-3.0, spread=0.1)
    check(p, device, batched=True)


def test_int32_saved_state(device):
    p = wl.cfg1(1)
    g64 = run_gpu(p, device)
    g32 = run_gpu(p, device, index_dtype=torch.int32)
    for a, b in zip(g64[3:], g32[3:]):
        grad_close(a, b, "int32 vs int64", rtol=1e-5)


@pytest.mark.parametrize("kind", ["last", "order", "negative", "range"])
@pytest.mark.parametrize("route", ["reduction", "one_launch"])
def test_saved_state_errors(kind, route, device):
    """The reference's saved-state errors from the drop-in backward, on both of its routes: without
    the forward workspace (reduction + finish) and with it (the training Function's route, the
    one-launch kernel for this small field), the kernels skipping the offending pairs."""
    p = tiny_problem(48, 48, 12, 12).to(device)
    delta, tp, ids, ws = ext.forward_with_workspace(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp,
                                                    16, 16, 3.0, False, 80.0)
    extra = {"forward_workspace": ws} if route == "one_launch" else {}
    if route == "one_launch":
        assert 0 <= ws.gf_max_span < 320
    tp, ids = tp.clone(), ids.clone()
    if kind == "last":
        tp[-1] += 1
        msg = "tile_ptr\\[-1\\] must equal"
    elif kind == "order":
        a, b = int(tp[1]), int(tp[2])
        tp[1] = b + 1  # tp[1] > tp[2]: decreasing
        tp[2] = a
        msg = "monotonic"
    elif kind == "negative":
        ids[0] = -3
        msg = "non-negative"
    else:
        ids[-1] = p.k + 5
        msg = "out-of-range"
    with pytest.raises(RuntimeError, match=msg):
        ext.gaussian_field_backward(p.grad, p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, tp,
                                    ids, 16, 16, 3.0, False, 80.0, **extra)
    torch.cuda.synchronize()


def test_autograd_train_function(device):
    """gaussian_field_train's forward and backward against the oracle, twice; the training
    Function's one-time backward notice (reference runtime.py:165-174) appears on the first
    backward only."""
    p = wl.cfg2(4)
    q = p.to(device)
    r = oracle(p)
    mu = q.mu.clone().requires_grad_(True)
    raw = q.chol_raw.clone().requires_grad_(True)
    amp = q.amp.clone().requires_grad_(True)
    runtime.GaussianFieldCudaTrainFunction._backward_warning_emitted = False
    notices = 0
    for attempt in range(2):
        for t in (mu, raw, amp):
            t.grad = None
        delta = runtime.gaussian_field_train(row_coords=q.row_coords, col_coords=q.col_coords, mu=mu,
                                             chol_raw=raw, amp=amp, tile_out=16, tile_in=16,
                                             sigma_multiplier=3.0, normalize=False, clamp_quad=80.0)
        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always")
            (delta * q.grad).sum().backward()
        torch.cuda.synchronize()
        notices += sum("gaussian_field_train uses the active custom CUDA backward path" in str(w.message)
                       for w in caught)
        assert notices == 1, f"attempt {attempt}: {notices} notices"
        assert runtime.GaussianFieldCudaTrainFunction._backward_warning_emitted
        field_close(delta, r[0])
        grad_close(mu.grad, r[3], "mu.grad")
        grad_close(raw.grad, r[4], "chol_raw.grad")
        grad_close(amp.grad, r[5], "amp.grad")


def _oracle_span(p: wl.FieldProblem, tile_out=16, tile_in=16, sigma=3.0) -> int:
    """The most tiles one Gaussian's rectangle covers, from the oracle's bounds (bounds.py:24-75)."""
    if p.k == 0:
        return 0
    b = fo.tile_bounds(p.mu, fo.activate_cholesky(p.chol_raw), p.out_features, p.in_features, tile_out, tile_in,
                       sigma)
    return int(b.tiles_touched.max())


def _wide(p: wl.FieldProblem, n: int) -> wl.FieldProblem:
    """p with its first n Gaussians spread over the whole grid."""
    p.chol_raw[:n, 0] = 4.0
    p.chol_raw[:n, 2] = 4.0
    return p


@pytest.mark.parametrize("case", ["cfg1", "cfg2", "cfg3", "cfg3_wide", "tile32", "emit_k9000", "k0", "ragged"])
def test_bin_info_matches_oracle(device, case):
    """gf_bin_info (P and the widest rectangle) from the binning's own read-back
    (gf_forward_bin_info, the drop-in forward) and from gf_read_bin_info after gf_forward, on
    each binning path: k_bin_tiles (cfg3, 32x32 tiles), binning in the render (cfg1, cfg2), the
    emission path (K past the masks) and K = 0: equal to the oracle's pair count and largest
    tiles_touched."""
    kw = {}
    if case == "cfg1":
        p = wl.cfg1(11)
    elif case == "cfg2":
        p = wl.cfg2(11)
    elif case == "cfg3":
        p = wl.cfg3(11)
    elif case == "cfg3_wide":
        p = _wide(wl.cfg3(11), 1)
    elif case == "tile32":
        p, kw = wl.cfg3(12), dict(tile_out=32, tile_in=32)
    elif case == "emit_k9000":
        p = wl.make_problem("emit_320_k9000", 320, 320, 9000, math.log(2.0), 0.5, 13)
    elif case == "k0":
        p = wl.make_problem("k0_64", 64, 64, 0, 0.0, 0.5, 14)
    else:
        p = wl.make_problem("ragged_333x517_k700", 333, 517, 700, math.log(6.0), 0.7, 15)
    to = kw.get("tile_out", 16)
    span = _oracle_span(p, to, to)
    P = int(fo.tile_bounds(p.mu, fo.activate_cholesky(p.chol_raw), p.out_features, p.in_features, to, to,
                           3.0).tiles_touched.sum()) if p.k else 0
    say(f"{case}: P={P} max_span={span}")
    q = p.to(device)
    plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=max(P, 1), **kw)
    plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    assert plan.bin_info() == (P, span)
    assert plan.status() == 0
    if p.k:
        _, tp, _, ws = ext.forward_with_workspace(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, to, to, 3.0,
                                                  False, 80.0)
        torch.cuda.synchronize()
        assert int(tp[-1]) == P and ws.gf_max_span == span


@pytest.mark.parametrize("case", ["cfg2", "cfg3", "cfg3_wide", "cfg3_int32"])
def test_train_backward_paths(device, case):
    """gaussian_field_train's backward (gf_backward_train): the one-launch kernel + slot move-out
    where the forward's binning allows it (cfg2 binned in the render, cfg3), the reduction +
    finish for a Gaussian over the whole grid (6400 tiles) and for int32 saved state.  Each
    against the oracle; a second backward through the same graph (retain_graph) returns the same
    gradients, so the move-out left the slots clear; and the gradients agree with the reduction
    path's (ext backward without the forward workspace) to fp32 rounding."""
    p = {"cfg2": lambda: wl.cfg2(21), "cfg3": lambda: wl.cfg3(21), "cfg3_wide": lambda: _wide(wl.cfg3(21), 1),
         "cfg3_int32": lambda: wl.cfg3(21)}[case]()
    r = oracle(p)
    P, span = int(r[1][-1]), _oracle_span(p)
    q = p.to(device)
    cfg = _native.make_config(16, 16, 3.0, False, 80.0)
    one = _native.lib().gf_backward_direct_launches(ctypes.byref(cfg), p.out_features, p.in_features, p.k, P,
                                                    span) == 1
    say(f"{case}: P={P} max_span={span} field takes the one-launch kernel: {one}")
    assert one == (case != "cfg3_wide")  # int32 saved state takes gf_backward all the same
    mu = q.mu.clone().requires_grad_(True)
    raw = q.chol_raw.clone().requires_grad_(True)
    amp = q.amp.clone().requires_grad_(True)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        if case == "cfg3_int32":
            # int32 saved state through the training Function's backward, as the reference permits
            delta, tp, ids, ws = ext.forward_with_workspace(q.row_coords, q.col_coords, mu, raw, amp, 16, 16, 3.0,
                                                            False, 80.0)
            grads = [ext.gaussian_field_backward(q.grad, q.row_coords, q.col_coords, mu.detach(), raw.detach(),
                                                 amp.detach(), tp.to(torch.int32), ids.to(torch.int32), 16, 16, 3.0,
                                                 False, 80.0, forward_workspace=ws) for _ in range(2)]
        else:
            delta = runtime.gaussian_field_train(row_coords=q.row_coords, col_coords=q.col_coords, mu=mu,
                                                 chol_raw=raw, amp=amp, tile_out=16, tile_in=16,
                                                 sigma_multiplier=3.0, normalize=False, clamp_quad=80.0)
            grads = []
            for _ in range(2):
                for t in (mu, raw, amp):
                    t.grad = None
                (delta * q.grad).sum().backward(retain_graph=True)
                grads.append([mu.grad.clone(), raw.grad.clone(), amp.grad.clone()])
    torch.cuda.synchronize()
    field_close(delta, r[0])
    for i, g in enumerate(grads):
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), g, r[3:]):
            grad_close(a, b, f"{name} (backward {i + 1})")
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), grads[1], grads[0]):
        grad_close(a, b, f"{name}, second backward vs first", rtol=1e-5)  # float atomics: not bit-equal
    _, tp, ids, ws = ext.forward_with_workspace(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, 16, 16, 3.0,
                                                False, 80.0)
    two = ext.gaussian_field_backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, tp, ids, 16, 16,
                                      3.0, False, 80.0)
    torch.cuda.synchronize()
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), grads[0], two):
        grad_close(a, b, f"{name} vs the reduction + finish", rtol=1e-5)


def test_stage2_validation_metadata(device):
    p = wl.cfg1(2)
    q = p.to(device)
    delta, meta = runtime.gaussian_field_cuda_field_stage2_validation(
        row_coords=q.row_coords, col_coords=q.col_coords, mu=q.mu, chol_raw=q.chol_raw, amp=q.amp,
        tile_out=16, tile_in=16, sigma_multiplier=3.0)
    ref_delta, ref_tp, ref_ids = fo.gaussian_field_forward(p.row_coords, p.col_coords, p.mu,
                                                           p.chol_raw, p.amp, 16, 16, 3.0)
    field_close(delta, ref_delta)
    binning_equal(meta["tile_ptr"], meta["gaussian_ids_sorted"], ref_tp, ref_ids)
    assert torch.equal(meta["per_tile_counts"].cpu(), ref_tp[1:] - ref_tp[:-1])
    assert meta["num_tile_rows"] == 20.0 and meta["num_tile_cols"] == 20.0
    assert meta["execution_mode"] == "cuda_field_stage2_validation"


def test_plan_sync_free_and_capacity(device):
    p = wl.cfg2(5)
    q = p.to(device)
    ref = run_gpu(p, device)
    P = int(ref[1][-1])
    plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P)
    plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P)
    torch.cuda.synchronize()
    assert plan.status() == 0 and plan.pairs() == P
    assert torch.equal(plan.delta, ref[0]) and torch.equal(plan.tile_ptr, ref[1])
    assert torch.equal(plan.ids[:P], ref[2])
    # same arithmetic; fp32 atomics accumulate the tiles in a run-dependent order
    for a, b in zip((plan.d_mu, plan.d_chol_raw, plan.d_amp), ref[3:]):
        grad_close(a, b, "plan", rtol=1e-5)
    # Gaussian constants recomputed from mu / chol_raw instead of reused from the forward.
    fresh = [t.clone() for t in plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw,
                                              q.amp, num_pairs=P, reuse_forward=False)]
    for a, b in zip(fresh, ref[3:]):
        # same arithmetic, different atomic accumulation order
        grad_close(a, b, "plan without the forward's constants", rtol=1e-5)
    small = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P // 2)
    small.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    torch.cuda.synchronize()
    assert small.status() & _native.GF_STATUS_CAPACITY


def _random_forward_problem(i: int):
    """Seeded 16x16-tile fields with 1 <= K <= 1024, most below 8 pairs per tile: ragged sizes,
    sub-pixel to whole-matrix Gaussians, indefinite covariances, normalisation, clamps, sigma."""
    g = torch.Generator().manual_seed(1000 + i)
    K = [1, 2, 63, 64, 65, 255, 256, 257, 511, 700, 1023, 1024][i % 12]
    lo, hi = (1, 300) if K <= 256 else (250, 720)  # more Gaussians on larger fields: < 8 pairs a tile
    M = int(torch.randint(lo, hi, (1,), generator=g))
    N = int(torch.randint(lo, hi, (1,), generator=g))
    log_px = float(torch.empty(1).uniform_(-1.0, 2.5, generator=g))
    spread = float(torch.empty(1).uniform_(0.0, 1.2, generator=g))
    p = wl.make_problem(f"rand_fwd_{i}_{M}x{N}_k{K}", M, N, K, log_px, spread, 2000 + i)
    if i % 5 == 3:  # elongated Gaussians whose fp32 covariance is indefinite
        nb = min(K, 3)
        bad = _indefinite_problem(max(M, 2), max(N, 2), 3000 + i, n_normal=1, n_bad=nb)
        p.chol_raw[:nb] = bad.chol_raw[1:]
    if i % 7 == 2:  # a few Gaussians covering the whole matrix
        p.chol_raw[: min(K, 5), 0] = 4.0
        p.chol_raw[: min(K, 5), 2] = 4.0
    cfg = dict(sigma=[3.0, 2.5, 1.5, 3.5][i % 4], normalize=i % 6 == 5, clamp=[80.0, 24.0, None, 200.0][i % 4])
    return p, cfg


@pytest.mark.parametrize("i", range(24))
def test_gf_forward_random_fields(device, i):
    """FieldPlan.forward (the one-call gf_forward) against the float64 evaluation and, bit for
    bit, against the forward called phase by phase (gf_forward_bin / _emit / _render): tile_ptr,
    ids, delta-W, the constants the backward reads, and the backward's gradients; then an id
    capacity below the pair count."""
    p, cfg = _random_forward_problem(i)
    r = fo.gaussian_field_fwd_bwd_batched(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, 16, 16,
                                          cfg["sigma"], cfg["normalize"], cfg["clamp"])
    P = int(r[1][-1])
    T = (-(-p.out_features // 16)) * (-(-p.in_features // 16))
    cap = max(P, 1)
    say(f"{p.name} P={P} T={T} {cfg}")
    q = p.to(device)
    kw = dict(sigma_multiplier=cfg["sigma"], normalize=cfg["normalize"], clamp_quad=cfg["clamp"])
    one = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=cap, **kw)
    phased = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=cap, **kw)
    one.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    phased.forward_phases(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    gf = [t.clone() for t in one.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P)]
    gp = [t.clone() for t in phased.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                             num_pairs=P)]
    torch.cuda.synchronize()
    assert one.status() == 0 and one.pairs() == P
    binning_equal(one.tile_ptr, one.ids[:P], r[1], r[2])
    assert torch.equal(one.tile_ptr, phased.tile_ptr) and torch.equal(one.ids[:P], phased.ids[:P])
    assert torch.equal(one.delta, phased.delta), "delta-W differs from the three-phase forward"
    n = 8 * p.k  # the constants the backward reads: eval[K] (32 B each) in both workspaces
    assert torch.equal(one.fwd_ws[256:256 + 4 * n], phased.fwd_ws[256:256 + 4 * n])
    # Random sizes and spreads give covariance condition numbers in the thousands, where no two
    # fp32 evaluation orders agree to 1e-5 (the fp32 oracle is itself up to 1.6e-5 from the
    # float64 evaluation); the yardstick is float64: at least as close to it as the oracle.
    r64 = fo.gaussian_field_fwd_bwd_fp64(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, 16, 16,
                                         cfg["sigma"], cfg["normalize"], cfg["clamp"])
    finite = torch.isfinite(r64[0])
    assert torch.equal(torch.isfinite(one.delta.cpu()), finite)  # NaN: normalised indefinite Gaussians
    if bool(finite.any()):
        scale = max(float(r64[0][finite].abs().max()), 1e-30)
        err_g = float((one.delta.cpu().double() - r64[0])[finite].abs().max()) / scale
        err_o = float((r[0].double() - r64[0])[finite].abs().max()) / scale
        assert err_g <= err_o + 1e-5, (err_g, err_o)
    for name, a, b, c, o in zip(("d_mu", "d_chol_raw", "d_amp"), gf, gp, r64[3:], r[3:]):
        fin = torch.isfinite(c)
        if not bool(fin.all()):
            continue
        grad_close(a, b, f"{name} vs three-phase", rtol=1e-5)
        cn = float(c.norm())
        if cn > 0.0:
            eg = float((a.cpu().double() - c).norm()) / cn
            eo = float((o.double() - c).norm()) / cn
            assert eg <= eo + 1e-4, (name, eg, eo)
    if P > 1:  # an id capacity below the pair count: status CAPACITY, tile_ptr and P complete
        small = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P // 2, **kw)
        small.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        torch.cuda.synchronize()
        assert small.status() & _native.GF_STATUS_CAPACITY and small.pairs() == P
        assert torch.equal(small.tile_ptr, one.tile_ptr)
        if int((one.tile_ptr[1:] - one.tile_ptr[:-1]).max()) <= HEAVY_TILE:
            # no heavy tile: both plans render every tile the same way
            assert torch.equal(small.delta, one.delta)
            assert torch.equal(small.ids[:P // 2], one.ids[:P // 2])
        # else the capacity bounds the heavy-tile workgroups too: past it, heavy tiles beyond the
        # bound may go unrendered (the status bit asks for a larger capacity; tile_ptr and P hold)


def _direct_vs_two_launch(plan, q, P, r64=None, r=None):
    """FieldPlan.backward_direct against FieldPlan.backward (reduction + finish) on the same
    forward; with r64 / r (float64 / fp32 oracle results) also against float64."""
    two = [t.clone() for t in plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                            num_pairs=P)]
    one = [t.clone() for t in plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                   num_pairs=P)]
    torch.cuda.synchronize()
    assert plan.status("backward") == 0
    errs = {}
    for k, (name, a, b) in enumerate(zip(("d_mu", "d_chol_raw", "d_amp"), one, two)):
        if r64 is not None:
            c = r64[3 + k]
            if not bool(torch.isfinite(c).all()):
                continue
            cn = float(c.norm())
            if cn > 0.0:
                ed = float((a.cpu().double() - c).norm()) / cn
                eo = float((r[3 + k].double() - c).norm()) / cn
                assert ed <= eo + 1e-4, (name, ed, eo)
        errs[name] = grad_close(a, b, f"{name}: direct vs two launches")
    return one, errs


@pytest.mark.parametrize("case", ["cfg1", "cfg2", "cfg3", "cfg3_clamp24", "cfg2_normalize", "cfg2_noclamp",
                                  "cfg3_tile32"])
def test_backward_direct_matches_oracle(device, case):
    """gf_backward_direct (the chain rule applied per tile with the maps k_prep stores, one
    launch) against the CPU oracle and against the reduction + finish, then a second forward
    with other parameters on the same plan (the forward clears the gradients the direct
    backward adds into)."""
    base, _, opt = case.partition("_")
    kw = {"clamp24": dict(clamp_quad=24.0), "normalize": dict(normalize=True), "noclamp": dict(clamp_quad=None),
          "tile32": dict(tile_out=32, tile_in=32), "": {}}[opt]
    okw = dict(tile_out=kw.get("tile_out", 16), tile_in=kw.get("tile_in", 16), normalize=kw.get("normalize", False),
               clamp=kw.get("clamp_quad", 80.0))
    for seed in (11, 12):
        p = getattr(wl, base)(seed)
        r = oracle(p, **okw)
        P = int(r[1][-1])
        say(f"{case} seed {seed}: M={p.out_features} N={p.in_features} K={p.k} P={P} {kw}")
        if seed == 11:
            plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P + 4096, **kw)
        q = p.to(device)
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        assert plan.direct_launches(P) == 1
        one, errs = _direct_vs_two_launch(plan, q, P)
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), one, r[3:]):
            errs[name + " vs oracle"] = grad_close(a, b, name)
        say("  ok " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))


@pytest.mark.parametrize("i", range(24))
def test_backward_direct_random_fields(device, i):
    """The direct backward on the seeded random fields of test_gf_forward_random_fields (ragged
    sizes, indefinite covariances through the general-form pass, normalisation, clamps 24 / 80 /
    200 / none, sigma 1.5..3.5): at least as close to the float64 evaluation as the fp32 oracle,
    and within 1e-4 of the reduction + finish."""
    p, cfg = _random_forward_problem(i)
    r = fo.gaussian_field_fwd_bwd_batched(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, 16, 16,
                                          cfg["sigma"], cfg["normalize"], cfg["clamp"])
    r64 = fo.gaussian_field_fwd_bwd_fp64(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, 16, 16,
                                         cfg["sigma"], cfg["normalize"], cfg["clamp"])
    P = int(r[1][-1])
    say(f"{p.name} P={P} {cfg}")
    q = p.to(device)
    plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=max(P, 1),
                     sigma_multiplier=cfg["sigma"], normalize=cfg["normalize"], clamp_quad=cfg["clamp"])
    plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    _direct_vs_two_launch(plan, q, P, r64, r)


@pytest.mark.parametrize("nbig", [1, 4, 16])
def test_backward_direct_hot_gaussians(device, nbig):
    """Gaussians over the whole grid (6,400 tiles each, every tile's atomics on their one slot) in
    the one-launch backward: against the oracle, then a second backward on the same forward
    adds the same gradients again (each doubles).  With 16 of them the tiles are dense and the
    call takes the striped reduction + finish, whose finish adds into the same slots: a second
    backward doubles them there too."""
    p = wl.cfg3(3)
    p.chol_raw[:nbig, 0] = 4.0
    p.chol_raw[:nbig, 2] = 4.0
    r = oracle(p)
    P = int(r[1][-1])
    say(f"cfg3 with {nbig} whole-grid Gaussians: P={P}")
    q = p.to(device)
    plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P)
    plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    one_launch = plan.direct_launches(P) == 1  # 16 such Gaussians make the tiles dense: the fallback
    once = [t.clone() for t in plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                    num_pairs=P)]
    torch.cuda.synchronize()
    assert plan.status() == 0 and plan.status("backward") == 0
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), once, r[3:]):
        grad_close(a, b, name)
    twice = plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P)
    torch.cuda.synchronize()
    # both paths add into the slots the forward cleared
    say(f"  second backward ({'one launch' if one_launch else 'reduction + finish'})")
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), twice, once):
        grad_close(a, 2.0 * b, f"{name} after a second backward", rtol=1e-5)
    big = twice[2][:nbig].abs().cpu()
    assert float(big.min()) > 0.0, "hot Gaussians' gradients missing"
    # with the widest rectangle known (6400 tiles) the call takes the reduction + finish
    P2, span = plan.bin_info()
    assert P2 == P and span == 6400 and plan.direct_launches(P, span) == 2
    plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    known = plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P,
                                 max_span=span)
    torch.cuda.synchronize()
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), known, r[3:]):
        grad_close(a, b, f"{name} (max_span known)")


def test_backward_direct_fallbacks(device):
    """Fields the one-launch kernel does not take run the reduction + finish into the direct
    gradients: FieldPlan.backward's kernels (equal up to the order of the float atomics).  Dense
    tiles (>= 16 pairs a tile), the emission path (K past the masks), 8x8 tiles, a grid of 8960
    tiles (8 accumulator stripes) whose widest rectangle is not given; K = 0."""
    cases = [
        (wl.make_problem("dense_320_k600", 320, 320, 600, math.log(24.0), 0.2, 31), {}),
        (wl.make_problem("emit_320_k9000", 320, 320, 9000, math.log(2.0), 0.5, 33), {}),
        (wl.make_problem("tile8_200_k100", 200, 200, 100, math.log(4.0), 0.5, 34), dict(tile_out=8, tile_in=8)),
        (wl.make_problem("stripes_1280x1792_k512", 1280, 1792, 512, math.log(8.0), 0.6, 36), {}),
        (wl.make_problem("k0_64", 64, 64, 0, 0.0, 0.5, 35), {}),
    ]
    for p, kw in cases:
        q = p.to(device)
        plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=max(1, 400 * p.k), **kw)
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        torch.cuda.synchronize()
        P = plan.pairs()
        T = plan.T
        say(f"{p.name}: P={P} T={T} {kw}")
        assert plan.status() == 0 and plan.direct_launches(P) == 2
        two = [t.clone() for t in plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                num_pairs=P)]
        one = plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P)
        torch.cuda.synchronize()
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), one, two):
            grad_close(a, b, name, rtol=1e-5)


def test_backward_direct_heavy_tiles_and_large_grids(device):
    """The one-launch backward on fields with heavy-tile workgroups (four waves a tile, their last
    rounds split over the slots) and on grids of 8192 tiles or more whose widest rectangle is
    known to be under 320 tiles: one launch, against the reduction + finish on the same forward
    (equal up to the order of the float atomics), twice in a row (the second call adds the same
    gradients again), and cfg5c's against the oracle."""
    cases = [
        wl.make_problem("heavy_640_k2048", 640, 640, 2048, math.log(6.0), 0.5, 32, clusters=4, cluster_sigma_px=30.0),
        wl.make_problem("stripes_1280x1792_k512", 1280, 1792, 512, math.log(8.0), 0.6, 36),
        wl.cfg5c(0),
    ]
    for p in cases:
        q = p.to(device)
        plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=max(1, 400 * p.k))
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        torch.cuda.synchronize()
        P, span = plan.bin_info()
        say(f"{p.name}: P={P} T={plan.T} widest rectangle {span}")
        assert plan.status() == 0 and span < 320 and plan.direct_launches(P, span) == 1
        two = [t.clone() for t in plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                num_pairs=P)]
        one = [t.clone() for t in plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw,
                                                       q.amp, num_pairs=P, max_span=span)]
        again = plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P,
                                     max_span=span)
        torch.cuda.synchronize()
        for name, a, b, c in zip(("d_mu", "d_chol_raw", "d_amp"), one, two, again):
            grad_close(a, b, name, rtol=1e-5)
            grad_close(c, 2.0 * b, f"{name} (second call)", rtol=1e-5)
        if p.name.startswith("cfg5c"):
            r = oracle(p, batched=True)
            for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), one, r[3:]):
                grad_close(a, b, f"{name} vs oracle")


def test_backward_both_reductions_between_8_and_16_pairs_a_tile(device):
    """Fields of 8 to 16 pairs a tile: the reduction + finish takes the transposing moment
    reduction there (from 8 pairs a tile), the one-launch backward still the row sums (up to 16).
    Both against the oracle and against each other (the order of the float atomics), with and
    without heavy-tile workgroups."""
    cases = [
        wl.make_problem("band_640_k900", 640, 640, 900, math.log(8.0), 0.5, 40),
        wl.make_problem("heavy_640_k2048", 640, 640, 2048, math.log(6.0), 0.5, 32, clusters=4, cluster_sigma_px=30.0),
    ]
    for p in cases:
        q = p.to(device)
        plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=max(1, 400 * p.k))
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        torch.cuda.synchronize()
        P, span = plan.bin_info()
        say(f"{p.name}: P={P} T={plan.T} ({P / plan.T:.2f} a tile) widest rectangle {span}")
        assert plan.status() == 0 and 8 * plan.T <= P < 16 * plan.T and plan.direct_launches(P, span) == 1
        two = [t.clone() for t in plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                num_pairs=P)]
        one = [t.clone() for t in plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw,
                                                       q.amp, num_pairs=P, max_span=span)]
        torch.cuda.synchronize()
        r = oracle(p, batched=True)
        for name, a, b, c in zip(("d_mu", "d_chol_raw", "d_amp"), one, two, r[3:]):
            grad_close(a, b, f"{name}: one launch vs reduction + finish", rtol=1e-5)
            grad_close(b, c, f"{name}: reduction + finish vs oracle")
            grad_close(a, c, f"{name}: one launch vs oracle")


def test_pair_render_unaligned_column_coordinates(device):
    """The pair renders' wave-wide fast paths (one aligned float4 of column coordinates a lane,
    the block sums and stores without per-lane tests) need a 16-byte aligned coordinate base; a
    column-coordinate view 4 bytes off takes the per-lane path.  ΔW, tile_ptr and ids bit-equal
    to the aligned call, for a single field on the mask path (the tile-pair kernel with
    heavy-tile workgroups) and for the same field as a batch layer (with its block sums)."""
    from guass_amd.ops import FieldBatchPlan

    p = wl.make_problem("unaligned_640_k2000", 640, 640, 2000, math.log(6.0), 0.5, 44)
    q = p.to(device)
    buf = torch.zeros(p.in_features + 1, device=device)
    buf[1:] = q.col_coords
    cc = buf[1:]
    assert cc.data_ptr() % 16 != 0 and torch.equal(cc, q.col_coords)
    cap = 400 * p.k
    outs = []
    for cols in (q.col_coords, cc):
        plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=cap)
        plan.forward(q.row_coords, cols, q.mu, q.chol_raw, q.amp)
        torch.cuda.synchronize()
        assert plan.status() == 0
        P = plan.pairs()
        outs.append((plan.delta.clone(), plan.tile_ptr.clone(), plan.ids[:P].clone()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    P = int(outs[0][1][-1])
    layers = [q, wl.FieldProblem(p.name + "_unaligned", p.out_features, p.in_features, q.row_coords, cc, q.mu,
                                 q.chol_raw, q.amp, q.grad)]
    batch = FieldBatchPlan(layers, device, capacities=[P, P])
    batch.forward()
    torch.cuda.synchronize()
    st, pairs, norms = batch.read(norms=True)
    assert st == [0, 0] and pairs == [P, P]
    a, b = batch.plans
    assert torch.equal(a.delta, b.delta) and torch.equal(a.ids[:P], b.ids[:P]) and norms[0] == norms[1]
    field_close(a.delta, outs[0][0], rtol=1e-6)  # the single field's heavy tiles sum in another order


def test_backward_stripes(device):
    """Tile grids of >= 2048 tiles spread each Gaussian's accumulators over 4 stripes (>= 8192: 8,
    >= 16384: 32): a 1280x1792 field (8960 tiles) against the oracle, alone and as a batch layer next to a
    one-stripe layer (the batched finish maps K * stripes threads per layer)."""
    from guass_amd.ops import FieldBatchPlan

    p = wl.make_problem("stripes8_1280x1792_k512", 1280, 1792, 512, math.log(8.0), 0.6, 21)
    g, r = check(p, device)
    small = wl.cfg2(22)
    singles = [run_gpu(small, device), g]
    batch = FieldBatchPlan([small.to(device), p.to(device)], device,
                           capacities=[int(sg[1][-1]) for sg in singles])
    batch.forward()
    batch.backward()
    torch.cuda.synchronize()
    assert batch.status() == [0, 0]
    for i, (pl, sg) in enumerate(zip(batch.plans, singles)):
        assert torch.equal(pl.delta, sg[0]), f"layer {i}: delta"
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), sg[3:]):
            grad_close(a, b, f"layer {i} {name}", rtol=1e-5)


def test_deterministic_forward(device):
    p = wl.cfg3(1)
    a = run_gpu(p, device)
    b = run_gpu(p, device)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])


def test_graph_replay_matches_eager(device):
    p = wl.cfg3(2)
    q = p.to(device)
    eager = run_gpu(p, device)
    P = int(eager[1][-1])
    plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P)
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P)
    torch.cuda.current_stream(device).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P)
    for rep in range(3):
        plan.delta.fill_(float("nan"))
        plan.d_mu.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(plan.delta, eager[0]), f"replay {rep}: delta"
        assert torch.equal(plan.ids[:P], eager[2]), f"replay {rep}: ids"
        for a, b in zip((plan.d_mu, plan.d_chol_raw, plan.d_amp), eager[3:]):
            grad_close(a, b, f"replay {rep}", rtol=1e-5)
        _ = (eager[0] * 2.0).sum().item()  # eager work between replays


def test_golden_fixture_tiny_ragged(device):
    """The committed fixture (tests/golden/tiny_ragged.npz) through the product path."""
    import numpy as np
    from pathlib import Path

    d = np.load(Path(__file__).resolve().parent / "golden" / "tiny_ragged.npz")
    t = lambda k: torch.from_numpy(d[k].copy()).to(device)  # noqa: E731
    say("golden tiny_ragged 45x70 K=12")
    delta, tp, ids = ext.gaussian_field_forward(t("row_coords"), t("col_coords"), t("mu"), t("chol_raw"),
                                                t("amp"), 16, 16, 3.0, False, 80.0)
    grads = ext.gaussian_field_backward(t("grad"), t("row_coords"), t("col_coords"), t("mu"),
                                        t("chol_raw"), t("amp"), tp, ids, 16, 16, 3.0, False, 80.0)
    torch.cuda.synchronize()
    binning_equal(tp, ids, torch.from_numpy(d["tile_ptr"]), torch.from_numpy(d["gaussian_ids"]))
    field_close(delta, torch.from_numpy(d["delta"]))
    for name, a in zip(("d_mu", "d_chol_raw", "d_amp"), grads):
        grad_close(a, torch.from_numpy(d[name]), name)


def _single_layer(p, device):
    """Forward + backward of one field through FieldPlan (sync-free path)."""
    q = p.to(device)
    ref = run_gpu(p, device)
    P = int(ref[1][-1])
    return ref, P


def test_batch_matches_single_layers(device):
    from guass_amd.ops import FieldBatchPlan

    k0 = tiny_problem(40, 56, 1, 13)
    k0.mu, k0.chol_raw, k0.amp = k0.mu[:0], k0.chol_raw[:0], k0.amp[:0]
    probs = [wl.cfg1(3), wl.cfg2(4), tiny_problem(45, 70, 12, 12), k0, wl.cfg1(5)]
    say("batch of " + ", ".join(f"{p.out_features}x{p.in_features}/K{p.k}" for p in probs))
    singles = [run_gpu(p, device) for p in probs]
    layers = [p.to(device) for p in probs]
    caps = [int(s[1][-1]) for s in singles]
    batch = FieldBatchPlan(layers, device, capacities=caps)
    batch.forward()
    batch.backward()
    torch.cuda.synchronize()
    assert batch.status() == [0] * len(probs)
    for i, (pl, s) in enumerate(zip(batch.plans, singles)):
        P = caps[i]
        assert torch.equal(pl.tile_ptr, s[1]), f"layer {i}: tile_ptr"
        assert torch.equal(pl.ids[:P], s[2]), f"layer {i}: ids"
        assert torch.equal(pl.delta, s[0]), f"layer {i}: delta"
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), s[3:]):
            grad_close(a, b, f"layer {i} {name}", rtol=1e-5)


def test_batch_tile_pairs_match_single_fields(device):
    """The batched render takes two horizontally adjacent 16x16 tiles a wave: the union of their
    Gaussians, staged once, with a zero amplitude on the tile that does not list one.  Per field
    configuration, a batch of the 24 seeded random fields (ragged sizes, odd tile-column counts,
    indefinite forms, clamps, normalisation, sub-pixel to whole-matrix Gaussians) plus two fields
    on the emission path (K > 8192; odd and even tile columns), against each field's
    single-field run: tile_ptr and ids bit for bit; delta-W bit for bit where no tile holds more
    than HEAVY_TILE Gaussians (beyond that the single-field render may split a tile over four waves, a
    different fp32 summation order: 1e-6 of the peak); the delta-W norm of the read-back; the
    gradients to 1e-4 of each other, each batch gradient at least as close to the float64
    evaluation as the single field's (+ 1e-5)."""
    from guass_amd.ops import FieldBatchPlan

    groups: dict = {}
    for i in range(24):
        p, cfg = _random_forward_problem(i)
        groups.setdefault((cfg["sigma"], cfg["normalize"], cfg["clamp"]), []).append(p)
    first = next(iter(groups))
    groups[first] += [tiny_problem(45, 70, 8300, 8), tiny_problem(60, 96, 9000, 9)]
    exact = odd = 0
    worst_gap = 0.0
    for (sigma, normalize, clamp), probs in groups.items():
        kw = dict(sigma=sigma, normalize=normalize, clamp=clamp)
        say(f"batch of {len(probs)} fields {kw}: " + ", ".join(f"{p.out_features}x{p.in_features}/K{p.k}"
                                                              for p in probs))
        singles = [run_gpu(p, device, **kw) for p in probs]
        caps = [max(int(sg[1][-1]), 1) for sg in singles]
        batch = FieldBatchPlan([p.to(device) for p in probs], device, capacities=caps, sigma_multiplier=sigma,
                               normalize=normalize, clamp_quad=clamp)
        batch.forward()
        batch.backward()
        st, pairs, norms = batch.read(norms=True)
        assert st == [0] * len(probs), st
        for i, (p, pl, sg) in enumerate(zip(probs, batch.plans, singles)):
            P = int(sg[1][-1])
            assert pairs[i] == P, f"{p.name}: pairs"
            assert torch.equal(pl.tile_ptr, sg[1]), f"{p.name}: tile_ptr"
            assert torch.equal(pl.ids[:P], sg[2]), f"{p.name}: ids"
            odd += (-(-p.in_features // 16)) % 2
            if int((sg[1][1:] - sg[1][:-1]).max()) <= HEAVY_TILE:
                exact += 1
                assert torch.equal(pl.delta.nan_to_num(7.0), sg[0].nan_to_num(7.0)), f"{p.name}: delta"
            else:
                # indefinite forms without a clamp overflow to +-inf in both renders, at the same pixels
                fin = torch.isfinite(sg[0])
                assert torch.equal(pl.delta[~fin].nan_to_num(7.0), sg[0][~fin].nan_to_num(7.0)), f"{p.name}: inf"
                field_close(pl.delta[fin], sg[0][fin], rtol=1e-6)
            want = float(torch.linalg.vector_norm(sg[0].double()))
            if math.isfinite(want):
                assert abs(norms[i] - want) <= 1e-6 * max(want, 1e-30), f"{p.name}: norm {norms[i]} vs {want}"
            else:
                assert not math.isfinite(norms[i]), f"{p.name}: norm {norms[i]} vs {want}"
            # gradients: the batch reduces its dense tiles with moments about each tile's first
            # column, the single field's sparse tiles about the Gaussian's centre -- two fp32
            # evaluations, each held to the float64 one
            r64 = fo.gaussian_field_fwd_bwd_fp64(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad,
                                                 16, 16, sigma, normalize, clamp)
            for name, a, b, c in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), sg[3:],
                                     r64[3:]):
                fin = torch.isfinite(b)
                assert torch.equal(torch.isfinite(a), fin), f"{p.name} {name}: non-finite entries differ"
                grad_close(a[fin], b[fin], f"{p.name} {name}", rtol=1e-4)
                if bool(torch.isfinite(c).all()) and float(c.norm()) > 0.0:
                    eb = float((a.cpu().double() - c).norm()) / float(c.norm())
                    es = float((b.cpu().double() - c).norm()) / float(c.norm())
                    worst_gap = max(worst_gap, eb - es)
                    assert eb <= es + 1e-5, (p.name, name, eb, es)
    say(f"  batch gradients at most {worst_gap:.1e} further from float64 than the single fields'")
    say(f"  {exact} of 26 fields bit-equal, {odd} with an odd tile-column count")
    assert exact >= 18 and odd >= 6  # 19 of 26 have no tile of more than HEAVY_TILE Gaussians


def test_dense_tiles_narrow_gaussians_against_float64(device):
    """Dense tiles (>= 16 pairs a tile), whose backward takes its moments about the tile's middle
    column and shifts them to the Gaussian's centre, on sub-pixel Gaussians (sigma 0.2-0.6 px):
    the shift cancels by up to (offset / sigma)^2, largest for narrow Gaussians near a tile's
    edge.  Random centres and centres on tile edges; the single-field kernel (P >= 16 T) and the
    batched one, each against the float64 evaluation of the reference program: at most 1e-5
    further from it than the fp32 oracle (measured: 1.3e-6 further; the gradient bar is 1e-4)."""
    from guass_amd.ops import FieldBatchPlan

    probs = []
    for seed, edges in ((71, False), (72, True)):
        p = wl.make_problem(f"narrow_dense_s{seed}{'_edges' if edges else ''}", 256, 256, 6000, math.log(0.35), 0.3,
                            seed)
        if edges:  # column centres half a pixel inside a tile's first or last column
            g = torch.Generator().manual_seed(seed)
            tcol = torch.randint(0, 16, (p.k,), generator=g).to(torch.float64)
            side = torch.randint(0, 2, (p.k,), generator=g).to(torch.float64)
            px = 16.0 * tcol + 0.5 + 14.0 * side
            p.mu[:, 1] = (2.0 * px / (p.in_features - 1) - 1.0).to(torch.float32)
        probs.append(p)
    worst = 0.0
    for p in probs:
        r = oracle(p, batched=True)
        P = int(r[1][-1])
        T = (-(-p.out_features // 16)) * (-(-p.in_features // 16))
        say(f"{p.name}: P={P} ({P / T:.1f} pairs a tile)")
        assert P >= 16 * T
        r64 = fo.gaussian_field_fwd_bwd_fp64(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, 16, 16, 3.0,
                                             False, 80.0)
        single = run_gpu(p, device)
        batch = FieldBatchPlan([p.to(device)], device, capacities=[P])
        batch.forward()
        batch.backward()
        torch.cuda.synchronize()
        assert batch.status() == [0]
        pl = batch.plans[0]
        for name, a, b, c, o in zip(("d_mu", "d_chol_raw", "d_amp"), single[3:], (pl.d_mu, pl.d_chol_raw, pl.d_amp),
                                    r64[3:], r[3:]):
            cn = float(c.norm())
            eo = float((o.double() - c).norm()) / cn
            es = float((a.cpu().double() - c).norm()) / cn
            eb = float((b.cpu().double() - c).norm()) / cn
            say(f"  {name}: oracle {eo:.2e}, single field {es:.2e}, batch {eb:.2e} from float64")
            worst = max(worst, es - eo, eb - eo)
            assert es <= eo + 1e-5 and eb <= eo + 1e-5, (p.name, name, eo, es, eb)
    say(f"  at most {worst:.1e} further from float64 than the oracle")


# One cfg4 layer of each of the six distinct SD1.5 attention shapes (index into
# wl.sd15_attention_shapes(): block 0 attn1.to_q 320x320, block 0 attn2.to_k 320x768, block 2
# attn1.to_q 640x640, block 2 attn2.to_k 640x768, block 4 attn1.to_q 1280x1280, block 4
# attn2.to_k 1280x768).
SD15_SHAPE_PICK = [0, 5, 16, 21, 32, 37]


def _cfg4_layer(i: int) -> wl.FieldProblem:
    """Layer i of wl.cfg4(0) (same seed, distribution and K = 1024) without drawing the others."""
    name, m, n = wl.sd15_attention_shapes()[i]
    return wl.make_problem(f"cfg4_{name}", m, n, 1024, math.log(8.0), 0.6, i)


def test_batch_sd15_layers_against_oracle(device):
    """One BASELINE cfg4 layer of each of the six SD1.5 attention shapes (320x320, 320x768,
    640x640, 640x768, 1280x1280, 1280x768; K = 1024 each) in one batch, against the CPU
    oracle."""
    from guass_amd.ops import FieldBatchPlan

    probs = [_cfg4_layer(i) for i in SD15_SHAPE_PICK]
    assert sorted({(p.out_features, p.in_features) for p in probs}) == sorted(
        {(m, n) for _, m, n in wl.sd15_attention_shapes()})
    refs = []
    for p in probs:
        say(f"  oracle {p.name} {p.out_features}x{p.in_features}")
        refs.append(oracle(p, batched=True))
    layers = [p.to(device) for p in probs]
    batch = FieldBatchPlan(layers, device, capacities=[int(r[1][-1]) for r in refs])
    batch.forward()
    batch.backward()
    torch.cuda.synchronize()
    assert batch.status() == [0] * len(probs)
    for p, pl, r in zip(probs, batch.plans, refs):
        say(f"  {p.name} {p.out_features}x{p.in_features}: pairs={int(r[1][-1])}")
        binning_equal(pl.tile_ptr, pl.ids[:int(r[1][-1])], r[1], r[2])
        field_close(pl.delta, r[0])
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), r[3:]):
            grad_close(a, b, name)


def test_batch_split_last_rounds(device):
    """A batch layer whose tiles hold 0..10 Gaussians (and 65, 66: second chunks of one and two),
    each Gaussian inside one tile: the batched backward takes a tile's last round of one or two
    Gaussians over all four slots (their columns split, the slots' moments added before the
    atomics). Binning, field and gradients against the CPU oracle."""
    from guass_amd.ops import FieldBatchPlan

    M = N = 80
    counts = [t % 11 for t in range(25)]
    counts[23], counts[24] = 65, 66
    g = torch.Generator().manual_seed(11)
    f64 = torch.float64
    centres = []
    for t, c in enumerate(counts):
        tr, tc = divmod(t, 5)
        base = torch.tensor([tr * 16 + 7.5, tc * 16 + 7.5], dtype=f64)
        centres.append(base + (torch.rand(c, 2, generator=g, dtype=f64) * 4.0 - 2.0))
    mean_px = torch.cat(centres)
    K = mean_px.shape[0]
    # sigma 0.8..1.25 px: the 3-sigma box of a centre within 2 px of the tile's middle stays inside the tile
    log_scale = 0.1 * torch.randn(K, 2, generator=g, dtype=f64).clamp(-2.0, 2.0)
    theta = torch.rand(K, generator=g, dtype=f64) * math.pi
    amp = torch.randn(K, generator=g, dtype=f64)
    mu, raw, amp32 = wl.pixel_to_params(M, N, mean_px, log_scale, theta, amp)
    rc, cc = wl.axes(M, N)
    grad = torch.randn(M * N, generator=g, dtype=f64).to(torch.float32)
    p = wl.FieldProblem("split_rounds", M, N, rc, cc, mu, raw, amp32, grad)
    say(f"split rounds: K={K} counts={counts}")
    r = oracle(p, batched=True)
    assert (r[1][1:] - r[1][:-1]).tolist() == counts  # one tile per Gaussian, as constructed
    batch = FieldBatchPlan([p.to(device)], device, capacities=[int(r[1][-1])])
    batch.forward()
    batch.backward()
    torch.cuda.synchronize()
    assert batch.status() == [0]
    pl = batch.plans[0]
    binning_equal(pl.tile_ptr, pl.ids[:int(r[1][-1])], r[1], r[2])
    field_close(pl.delta, r[0])
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), r[3:]):
        grad_close(a, b, name)


def test_batch_layers_narrower_than_a_tile(device):
    """Layers with fewer rows or columns than the 16x16 tile (one tile row or column; the tile is
    clamped to the matrix, which takes them off the mask path) in a batch with an ordinary
    layer: each renders tile by tile from emitted ids, against the CPU oracle (they used to be
    planned for the tile-pair render, which found no mask words: delta-W zero, status
    COUNT_MISMATCH)."""
    from guass_amd.ops import FieldBatchPlan

    specs = [("rows2", 2, 120, 300, 5062, 1, 3.0), ("cols10", 368, 10, 2500, 5049, 0, math.log(3.0)),
             ("tiny", 3, 5, 7, 11, 0, 0.0), ("plain", 64, 80, 200, 12, 0, math.log(4.0))]
    probs = [wl.make_problem(n, M, N, K, ls, 0.5, seed, clusters=cl, cluster_sigma_px=max(4.0, 0.05 * min(M, N)))
             for n, M, N, K, seed, cl, ls in specs]
    refs = [oracle(p, batched=True) for p in probs]
    batch = FieldBatchPlan([p.to(device) for p in probs], device, capacities=[max(1, int(r[1][-1])) for r in refs])
    batch.forward()
    batch.backward()
    torch.cuda.synchronize()
    assert batch.status() == [0] * len(probs)
    for p, pl, r in zip(probs, batch.plans, refs):
        say(f"  {p.name} {p.out_features}x{p.in_features} K={p.k}: pairs={int(r[1][-1])}")
        binning_equal(pl.tile_ptr, pl.ids[:int(r[1][-1])], r[1], r[2])
        field_close(pl.delta, r[0])
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), r[3:]):
            grad_close(a, b, name)


def test_random_fields_sweep(device):
    """40 seeded random fields (ragged sizes from 1 to 520, K from 0 to 2500, tiles 16, 32, 8, 24
    and mixed, normalisation, clamp 24 / 80 / 200 / none, clustered means, int32 and int64 ids)
    through the drop-in path against the CPU oracle; then the 16x16 fields, and the 32x32 fields
    of at least 32 rows and columns, as batches per clamp, against their single-field runs."""
    import random

    from guass_amd.ops import FieldBatchPlan

    rng = random.Random(4242)
    groups = {}
    for case in range(40):
        s = 4242 + case
        M, N = rng.randint(1, 520), rng.randint(1, 520)
        K = rng.choice([0, 1, 5, 63, 64, 65, 300, 1024, 2500])
        tile = rng.choice([16, 16, 16, 32, 8, 24])
        tile_in = tile if rng.random() < 0.8 else rng.choice([16, 32])
        normalize = rng.random() < 0.3
        clamp = rng.choice([80.0, 80.0, 200.0, 24.0, None])
        clusters = rng.choice([0, 0, 1, 3])
        ls = math.log(rng.choice([0.4, 1.0, 3.0, 8.0, 20.0]))
        idx = rng.choice([torch.int64, torch.int32])
        p = wl.make_problem(f"sweep{s}", M, N, K, ls, 0.5, s, clusters=clusters,
                            cluster_sigma_px=max(4.0, 0.05 * min(M, N)))
        kw = dict(tile_out=tile, tile_in=tile_in, normalize=normalize, clamp=clamp, index_dtype=idx)
        say(f"case {case}: M={M} N={N} K={K} {kw} clusters={clusters} log-scale {ls:.2f}")
        g = run_gpu(p, device, **kw)
        r = oracle(p, **{k: v for k, v in kw.items() if k != "index_dtype"})
        binning_equal(g[1], g[2], r[1], r[2])
        field_close(g[0], r[0])
        if K:
            for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), g[3:], r[3:]):
                grad_close(a, b, name)
        eligible = K > 0 and tile == tile_in and clamp is not None and not normalize and (
            tile == 16 or (tile == 32 and M >= 32 and N >= 32))
        if eligible:
            groups.setdefault((tile, clamp), []).append((p, g))
    for (tile, clamp), items in groups.items():
        say(f"batch of {len(items)} fields, tile {tile}, clamp {clamp}")
        batch = FieldBatchPlan([p.to(device) for p, _ in items], device,
                               capacities=[max(1, int(g[1][-1])) for _, g in items], tile_out=tile,
                               tile_in=tile, clamp_quad=clamp)
        batch.forward()
        batch.backward()
        torch.cuda.synchronize()
        assert batch.status() == [0] * len(items)
        for (p, g), pl in zip(items, batch.plans):
            P = int(g[1][-1])
            binning_equal(pl.tile_ptr, pl.ids[:P], g[1].cpu(), g[2].cpu())
            field_close(pl.delta, g[0].cpu())
            for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), g[3:]):
                grad_close(a, b.cpu(), name)


def test_cfg4_full_batch_matches_single_fields(device):
    """BASELINE cfg4 at its workload: all 128 SD1.5 attention layers (K = 1024 each) as one
    FieldBatchPlan, forward and backward, against each layer's own single-field run (the drop-in
    ext path; reference: each adapted layer renders its own delta-W, gaussian_linear.py:162-220).
    Binning is bit-equal for every layer.  delta-W is bit-equal where the single-field render
    has no heavy-tile workgroups; a field of >= 8 pairs per tile (the 320- and 640-wide layers,
    12-53 pairs per tile) renders its tiles of more than HEAVY_TILE Gaussians with four waves whose
    partial sums wave 0 adds, a different fp32 summation order from the batch's one wave per
    tile, so there delta-W agrees to 1e-6 of the field's peak.  Gradients agree to the atomics'
    summation order."""
    from guass_amd.ops import FieldBatchPlan

    probs = wl.cfg4(0)
    assert len(probs) == 128
    say(f"cfg4: 128 layers, sum M*N = {sum(p.out_features * p.in_features for p in probs)}")
    singles = []
    for i, p in enumerate(probs):
        singles.append(run_gpu(p, device))
        if i % 32 == 31:
            say(f"  single-field runs: {i + 1}/128")
    layers = [p.to(device) for p in probs]
    caps = [int(s[1][-1]) for s in singles]
    batch = FieldBatchPlan(layers, device, capacities=caps)
    tiles = [(-(-p.out_features // 16)) * (-(-p.in_features // 16)) for p in probs]
    assert batch.info.tile_blocks == sum(-(-t // 4) for t in tiles)  # four 16x16 tiles a workgroup
    pairs_of = [(-(-p.out_features // 16)) * -(-(-(-p.in_features // 16)) // 2) for p in probs]
    assert batch.info.render_blocks == sum(-(-t // 4) for t in pairs_of)  # four tile pairs a workgroup
    assert batch.info.tile_render == 0  # every layer renders by tile pairs
    batch.forward()
    batch.backward()
    torch.cuda.synchronize()
    st, pairs = batch.read()
    assert st == [0] * 128, [(i, x) for i, x in enumerate(st) if x]
    assert pairs == caps
    say(f"  batch done: {sum(caps)} pairs")
    exact = heavy = 0
    worst = 0.0
    for i, (pl, sg, t) in enumerate(zip(batch.plans, singles, tiles)):
        P = caps[i]
        assert torch.equal(pl.tile_ptr, sg[1]), f"layer {i}: tile_ptr"
        assert torch.equal(pl.ids[:P], sg[2]), f"layer {i}: ids"
        if P >= 8 * t:  # the single-field render split its heavy tiles over four waves
            heavy += 1
            worst = max(worst, field_close(pl.delta, sg[0], rtol=1e-6))
        else:
            exact += 1
            assert torch.equal(pl.delta, sg[0]), f"layer {i}: delta"
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), sg[3:]):
            grad_close(a, b, f"layer {i} {name}", rtol=1e-5)
    say(f"  every layer matches its single-field run: {exact} bit-equal, {heavy} heavy-tile layers "
        f"within {worst:.1e} of the peak")
    assert exact >= 48 and heavy >= 48


def _layers_from_problems(probs, device, tile=16):
    """GaussianLinear layers (K of each problem) holding the problems' parameters: mu_raw =
    atanh(mu) as the layer stores it, and the problems' CPU linspace axes."""
    from guass_amd.layers import GaussianAdapterConfig, GaussianLinear

    layers = []
    for p in probs:
        cfg = GaussianAdapterConfig(init_num_gaussians=p.k, tile_out=tile, tile_in=tile)
        ly = GaussianLinear(p.in_features, p.out_features, adapter_config=cfg, device=device)
        with torch.no_grad():
            ly.row_coords.copy_(p.row_coords.to(device))
            ly.col_coords.copy_(p.col_coords.to(device))
        ly.load_adapter_state({"mu_raw": torch.atanh(p.mu.clamp(-0.999999, 0.999999)),
                               "chol_raw": p.chol_raw, "amp": p.amp})
        layers.append(ly)
    return layers


def test_gaussian_field_batch_against_oracle(device):
    """GaussianFieldBatch.render() + autograd (the batched kernels take mu = tanh(mu_raw) and
    return dL/d(mu_raw)) against the CPU oracle's autograd through torch.tanh
    (gaussian_linear.py:153-154,178-190), on a cfg2 layer and a 1280x1280 cfg4 layer in one
    batch.  The oracle's forward uses the device's tanh values (torch's GPU tanh, the function
    the kernels call), which are checked against the CPU's to 1 ulp."""
    from guass_amd.layers import GaussianFieldBatch

    probs = [wl.cfg2(0), _cfg4_layer(32)]
    layers = _layers_from_problems(probs, device)
    fb = GaussianFieldBatch(layers)
    deltas = fb.render()
    torch.autograd.backward(deltas, [p.grad.to(device).view(p.out_features, p.in_features) for p in probs])
    torch.cuda.synchronize()
    for p, ly, d in zip(probs, layers, deltas):
        say(f"  {p.name} {p.out_features}x{p.in_features} K={p.k}: batched render vs oracle through tanh")
        mu_raw = ly.mu_raw.detach().cpu()
        mu_dev = torch.tanh(ly.mu_raw.detach()).cpu()
        ulp = (mu_dev.view(torch.int32) - torch.tanh(mu_raw).view(torch.int32)).abs().max()
        assert int(ulp) <= 1, f"device tanh {int(ulp)} ulp from the CPU's"
        r = fo.gaussian_linear_fwd_bwd(ly.row_coords.cpu(), ly.col_coords.cpu(), mu_raw, ly.chol_raw.detach().cpu(),
                                       ly.amp.detach().cpu(), p.grad, 16, 16, 3.0, False, 80.0,
                                       mu_values=mu_dev, batched=p.k > 256)
        pl = fb._plan.plans[layers.index(ly)]
        binning_equal(pl.tile_ptr, pl.ids[:int(r[1][-1])], r[1], r[2])
        field_close(d.detach().reshape(-1), r[0])
        for name, got, want in zip(("d_mu_raw", "d_chol_raw", "d_amp"), (ly.mu_raw.grad, ly.chol_raw.grad, ly.amp.grad),
                                   r[3:]):
            grad_close(got, want, name)


def test_batched_step_reads_back_once(device, monkeypatch):
    """A training step through GaussianFieldBatch -- render(), every layer's forward, autograd's
    backward -- makes one host read-back (FieldBatchPlan.read, which returns every layer's
    status, pair count and ||delta-W||) and no synchronising torch call (CUDA sync debug mode
    "error"); the reference synchronises per layer for delta_w_norm (gaussian_linear.py:218).
    Each layer's delta_w_norm metadata equals the norm of its delta-W to 1e-6."""
    from guass_amd.layers import GaussianFieldBatch
    from guass_amd.ops import FieldBatchPlan

    probs = [wl.cfg2(1), wl.cfg1(2), _cfg4_layer(16)]
    layers = _layers_from_problems(probs, device)
    fb = GaussianFieldBatch(layers)
    gen = torch.Generator(device=device).manual_seed(4)
    xs = [torch.randn(9, p.in_features, device=device, generator=gen) for p in probs]
    gys = [torch.randn(9, p.out_features, device=device, generator=gen) for p in probs]

    def step():
        fb.render()
        torch.autograd.backward([ly(x) for ly, x in zip(layers, xs)], gys)

    step()  # plans (uploading the plan synchronises)
    torch.cuda.synchronize()
    reads = []
    real_read = FieldBatchPlan.read

    def counting_read(self, *a, **kw):
        reads.append(kw)
        return real_read(self, *a, **kw)

    monkeypatch.setattr(FieldBatchPlan, "read", counting_read)
    for ly in layers:
        for t in (ly.mu_raw, ly.chol_raw, ly.amp):
            t.grad = None
    torch.cuda.set_sync_debug_mode("error")
    try:
        step()
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    say(f"  one step: {len(reads)} read-back(s)")
    assert len(reads) == 1
    for i, (ly, pl) in enumerate(zip(layers, fb._plan.plans)):
        meta = ly.last_forward_metadata
        assert meta["accumulate_backend"] == "batched_fields"
        want = float(pl.delta.double().norm())
        assert abs(meta["delta_w_norm"] - want) <= 1e-6 * want, (i, meta["delta_w_norm"], want)
        assert ly.amp.grad is not None and float(ly.amp.grad.abs().max()) > 0.0


def test_gaussian_field_reference_entry(device):
    """The validation entry gaussian_field_reference (runtime.py:236-270) with
    allow_reference_backward=True and the extension's gaussian_field_backward_reference
    (ext.cpp:73-110) at cfg2: delta-W and gradients against the oracle, the one-time warning of
    its backward (runtime.py:66-73), and the guard's RuntimeError without the flag."""

    p = wl.cfg2(0)
    q = p.to(device)
    r = oracle(p)
    mu = q.mu.clone().requires_grad_(True)
    raw = q.chol_raw.clone().requires_grad_(True)
    amp = q.amp.clone().requires_grad_(True)
    kw = dict(row_coords=q.row_coords, col_coords=q.col_coords, tile_out=16, tile_in=16, sigma_multiplier=3.0,
              normalize=False, clamp_quad=80.0)
    with pytest.raises(RuntimeError, match="gaussian_field_reference is validation-only"):
        runtime.gaussian_field_reference(mu=mu, chol_raw=raw, amp=amp, **kw)
    runtime.GaussianFieldCudaReferenceFunction._backward_warning_emitted = False
    for attempt in range(2):
        for t in (mu, raw, amp):
            t.grad = None
        delta = runtime.gaussian_field_reference(mu=mu, chol_raw=raw, amp=amp, allow_reference_backward=True, **kw)
        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always")
            (delta * q.grad).sum().backward()
        torch.cuda.synchronize()
        msgs = [str(w.message) for w in caught if "validation-only reference replay" in str(w.message)]
        assert len(msgs) == (1 if attempt == 0 else 0), msgs
        say(f"  gaussian_field_reference attempt {attempt}: warnings {len(msgs)}")
        field_close(delta, r[0])
        grad_close(mu.grad, r[3], "d_mu")
        grad_close(raw.grad, r[4], "d_chol_raw")
        grad_close(amp.grad, r[5], "d_amp")
    # the extension's entry directly, on int32 saved state
    _, tp, ids = ext.gaussian_field_forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, 16, 16, 3.0,
                                            False, 80.0)
    got = ext.gaussian_field_backward_reference(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                tp.to(torch.int32), ids.to(torch.int32), 16, 16, 3.0, False, 80.0)
    torch.cuda.synchronize()
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), got, r[3:]):
        grad_close(a, b, f"backward_reference {name}")


def test_batch_graph_replay(device):
    from guass_amd.ops import FieldBatchPlan

    probs = [wl.cfg1(7), wl.cfg2(8)]
    singles = [run_gpu(p, device) for p in probs]
    layers = [p.to(device) for p in probs]
    batch = FieldBatchPlan(layers, device, capacities=[int(s[1][-1]) for s in singles])
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        batch.forward()
        batch.backward()
    torch.cuda.current_stream(device).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        batch.forward()
        batch.backward()
    for rep in range(3):
        for pl in batch.plans:
            pl.delta.fill_(float("nan"))
            pl.d_amp.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i, (pl, sg) in enumerate(zip(batch.plans, singles)):
            assert torch.equal(pl.delta, sg[0]), f"replay {rep} layer {i}: delta"
            grad_close(pl.d_amp, sg[5], f"replay {rep} layer {i}: d_amp", rtol=1e-5)
        _ = sum(float(pl.delta.abs().sum()) for pl in batch.plans)  # eager work between replays


@pytest.mark.parametrize("tile", [16, 32])
def test_gaussian_linear_layer(device, tile):
    """GaussianLinear.compute_delta_weight / forward (gaussian_linear.py:162-253): delta-W and the
    gradients of mu_raw (through tanh), chol_raw and amp against the oracle; the row-chunked
    forward against the dense x (W + delta-W)^T + b."""
    import torch.nn.functional as F

    from guass_amd.layers import GaussianAdapterConfig, GaussianLinear

    say(f"GaussianLinear 96->80, K=48, tiles {tile}x{tile}")
    gen = torch.Generator().manual_seed(tile)
    cfg = GaussianAdapterConfig(init_num_gaussians=48, init_method="random_uniform", tile_out=tile,
                                tile_in=tile, adapter_scale=0.5, init_amp_scale=1e-2)
    base = torch.nn.Linear(96, 80, device=device)
    layer = GaussianLinear.from_linear(base, cfg)
    with torch.no_grad():  # varied sizes (sigma ~ 1.5-8 px) and orientations, well conditioned
        raw = torch.randn(48, 3, generator=gen)
        raw[:, 0] = raw[:, 0] * 0.5 - 2.5
        raw[:, 2] = raw[:, 2] * 0.5 - 2.5
        raw[:, 1] = raw[:, 1] * 0.03
        layer.chol_raw.copy_(raw.to(device))
    dW = layer.compute_delta_weight()
    G = torch.randn(80, 96, generator=gen).to(device)
    (dW * G).sum().backward()
    torch.cuda.synchronize()
    mu = layer.materialize_mu().detach().cpu()  # the same fp32 means the layer rendered
    ref = fo.gaussian_field_fwd_bwd(layer.row_coords.cpu(), layer.col_coords.cpu(), mu,
                                    layer.chol_raw.detach().cpu(), layer.amp.detach().cpu(),
                                    (0.5 * G).reshape(-1).cpu(), tile, tile, 3.0, False, 80.0)
    field_close(dW.detach().reshape(-1) / 0.5, ref[0])
    grad_close(layer.mu_raw.grad, ref[3] * (1.0 - mu * mu), "d_mu_raw")
    grad_close(layer.chol_raw.grad, ref[4], "d_chol_raw")
    grad_close(layer.amp.grad, ref[5], "d_amp")
    meta = layer.last_forward_metadata
    assert meta["execution_mode"] == "cuda_field_train"
    assert abs(meta["delta_w_norm"] - float(ref[0].double().norm())) <= 1e-5 * meta["delta_w_norm"]
    x = torch.randn(5, 96, generator=gen).to(device)
    with torch.no_grad():
        y = layer(x)
        assert layer.last_forward_metadata["delta_apply_row_chunk"] == float(min(80, max(tile, 64)))
        assert layer.last_forward_metadata["linear_composition"] == "base_plus_delta_row_chunk_accumulate"
        want = F.linear(x, layer.weight + layer.compute_delta_weight(), layer.bias)
    assert float((y - want).abs().max()) <= 1e-5 * float(want.abs().max())


@pytest.mark.parametrize("tile", [16, 32])
def test_gaussian_field_batch_matches_per_layer(device, tile):
    """GaussianFieldBatch.render() (one batched launch per phase for every layer, autograd
    through it) against each GaussianLinear rendering its own delta-W, over two training steps
    (parameters updated in between) with layers of different shapes and one layer whose forward
    does not run in the second step (zero dL/d(delta-W))."""
    import copy

    from guass_amd.layers import GaussianAdapterConfig, GaussianFieldBatch, GaussianLinear

    torch.manual_seed(7)
    shapes = [(96, 80, 48), (64, 64, 24), (120, 40, 36)]  # (in, out, K)
    layers_a, layers_b = [], []
    for i, (n_in, n_out, k) in enumerate(shapes):
        cfg = GaussianAdapterConfig(init_num_gaussians=k, tile_out=tile, tile_in=tile, adapter_scale=0.5,
                                    init_amp_scale=1e-2)
        la = GaussianLinear(n_in, n_out, adapter_config=cfg, device=device)
        with torch.no_grad():
            la.chol_raw.add_(torch.randn_like(la.chol_raw) * 0.2)
        layers_a.append(la)
        layers_b.append(copy.deepcopy(la))
    say("GaussianFieldBatch over 3 layers vs per-layer rendering, 2 steps")
    fb = GaussianFieldBatch(layers_b)
    xs = [torch.randn(6, n_in, device=device) for (n_in, _, _) in shapes]
    for step in range(2):
        used = [0, 1, 2] if step == 0 else [0, 2]
        for ls in (layers_a, layers_b):
            for ly in ls:
                for p in (ly.mu_raw, ly.chol_raw, ly.amp):
                    p.grad = None
        loss_a = sum((layers_a[i](xs[i]) ** 2).sum() for i in used)
        loss_a.backward()
        fb.render()
        outs_b = {i: layers_b[i](xs[i]) for i in used}
        loss_b = sum((outs_b[i] ** 2).sum() for i in used)
        loss_b.backward()
        torch.cuda.synchronize()
        for i in used:
            assert layers_b[i].last_forward_metadata["accumulate_backend"] == "batched_fields"
            na = layers_a[i].last_forward_metadata["delta_w_norm"]  # torch's norm().item()
            nb = layers_b[i].last_forward_metadata["delta_w_norm"]  # the batch's read-back
            assert abs(nb - na) <= 1e-6 * na, (step, i, na, nb)
            with torch.no_grad():
                ya = layers_a[i](xs[i])
            assert torch.equal(outs_b[i].detach(), ya), f"step {step} layer {i}: output"
        for i in range(3):
            for name in ("mu_raw", "chol_raw", "amp"):
                ga = getattr(layers_a[i], name).grad
                gb = getattr(layers_b[i], name).grad
                if i not in used:
                    assert ga is None and gb is not None and float(gb.abs().max()) == 0.0
                    continue
                grad_close(gb, ga, f"step {step} layer {i} {name}", rtol=1e-5)
        with torch.no_grad():  # an optimiser step, then the same parameters on both copies
            for la, lb in zip(layers_a, layers_b):  # (the gradients agree to atomic order only)
                for name in ("mu_raw", "chol_raw", "amp"):
                    pa, pb = getattr(la, name), getattr(lb, name)
                    if pa.grad is not None:
                        pa.add_(pa.grad, alpha=-0.05)
                    pb.copy_(pa)


@pytest.mark.skip(reason="kept off the GPU: capturing this step (autograd with the layers' hipBLASLt GEMMs "
                         "around the batched field kernels) ended the host process with a segmentation fault "
                         "in torch.cuda.graph's capture_end; no cause in this library's code has been shown")
def test_gaussian_field_batch_graph_step(device):
    """A training step through GaussianFieldBatch (render(check=False), the layers' forwards,
    autograd's backward) captured in a HIP graph and replayed three times, with eager work,
    cleared outputs and synchronisations between the replays: every replay's delta-W and
    gradients against an eager step on the same parameters; check() then reads back once."""
    from guass_amd.layers import GaussianAdapterConfig, GaussianFieldBatch, GaussianLinear

    torch.manual_seed(5)
    shapes = [(96, 80, 48), (64, 64, 24), (120, 40, 36), (160, 96, 64)]  # (in, out, K)
    layers = []
    for n_in, n_out, k in shapes:
        cfg = GaussianAdapterConfig(init_num_gaussians=k, tile_out=16, tile_in=16, adapter_scale=0.5,
                                    init_amp_scale=1e-2)
        ly = GaussianLinear(n_in, n_out, adapter_config=cfg, device=device)
        with torch.no_grad():
            ly.chol_raw.add_(torch.randn_like(ly.chol_raw) * 0.2)
        layers.append(ly)
    named = [(f"layer {i} {n}", getattr(ly, n)) for i, ly in enumerate(layers) for n in ("mu_raw", "chol_raw", "amp")]
    xs = [torch.randn(6, n_in, device=device) for n_in, _, _ in shapes]
    gys = [torch.randn(6, n_out, device=device) for _, n_out, _ in shapes]
    fb = GaussianFieldBatch(layers)

    def step(check):
        deltas = fb.render(check=check)
        torch.autograd.backward([ly(x) for ly, x in zip(layers, xs)], gys)
        return deltas

    with pytest.raises(RuntimeError, match="earlier checked render"):
        fb.render(check=False)  # no plan yet
    say("GaussianFieldBatch step in a HIP graph: eager reference")
    for _, t in named:
        t.grad = None
    ref_d = [d.detach().clone() for d in step(True)]
    ref_g = [t.grad.clone() for _, t in named]
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):  # warm-up of the unchecked step off the default stream
        for _ in range(2):
            for _, t in named:
                t.grad = None
            step(False)
    torch.cuda.current_stream(device).wait_stream(stream)
    torch.cuda.synchronize()
    for _, t in named:
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        deltas = step(False)
    torch.cuda.synchronize()
    for rep in range(3):
        say(f"  replay {rep}")
        junk = torch.randn(1 << 16, device=device)
        float(junk.sum())  # eager work and a synchronisation between the replays
        with torch.no_grad():
            for d in deltas:
                d.fill_(float("nan"))
            for _, t in named:
                t.grad.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (d, r) in enumerate(zip(deltas, ref_d)):
            assert torch.equal(d, r), f"replay {rep} layer {i}: delta-W"
        for (name, t), r in zip(named, ref_g):
            grad_close(t.grad, r, f"replay {rep} {name}", rtol=1e-5)
    pairs = fb.check()
    assert len(pairs) == len(layers) and all(n > 0 for n in pairs)


def test_gaussian_field_batch_unchecked_render(device):
    """render(check=False) skips the read-back and renders with the plan of the last checked
    render: over two eager steps its delta-W equals the checked render's and its gradients agree;
    check() reads back afterwards; an unchecked render without a plan, or after the parameter
    tensors changed, raises."""
    from guass_amd.layers import GaussianAdapterConfig, GaussianFieldBatch, GaussianLinear

    torch.manual_seed(5)
    shapes = [(96, 80, 48), (64, 64, 24), (120, 40, 36)]  # (in, out, K)
    layers = []
    for n_in, n_out, k in shapes:
        cfg = GaussianAdapterConfig(init_num_gaussians=k, tile_out=16, tile_in=16, adapter_scale=0.5,
                                    init_amp_scale=1e-2)
        ly = GaussianLinear(n_in, n_out, adapter_config=cfg, device=device)
        with torch.no_grad():
            ly.chol_raw.add_(torch.randn_like(ly.chol_raw) * 0.2)
        layers.append(ly)
    named = [(f"layer {i} {n}", getattr(ly, n)) for i, ly in enumerate(layers) for n in ("mu_raw", "chol_raw", "amp")]
    xs = [torch.randn(6, n_in, device=device) for n_in, _, _ in shapes]
    gys = [torch.randn(6, n_out, device=device) for _, n_out, _ in shapes]
    fb = GaussianFieldBatch(layers)

    def step(check):
        for _, t in named:
            t.grad = None
        deltas = [d.detach().clone() for d in fb.render(check=check)]
        torch.autograd.backward([ly(x) for ly, x in zip(layers, xs)], gys)
        torch.cuda.synchronize()
        return deltas, [t.grad.clone() for _, t in named]

    with pytest.raises(RuntimeError, match="earlier checked render"):
        fb.render(check=False)
    ref_d, ref_g = step(True)
    norms = [ly.last_forward_metadata["delta_w_norm"] for ly in layers]
    for rep in range(2):
        d, g = step(False)
        for i, (a, b) in enumerate(zip(d, ref_d)):
            assert torch.equal(a, b), f"unchecked render {rep} layer {i}: delta-W"
        for (name, _), a, b in zip(named, g, ref_g):
            grad_close(a, b, f"unchecked render {rep} {name}", rtol=1e-5)
        # the norm metadata is the last checked render's
        assert [ly.last_forward_metadata["delta_w_norm"] for ly in layers] == norms
    pairs = fb.check()
    assert len(pairs) == len(layers) and all(n > 0 for n in pairs)
    with torch.no_grad():  # new parameter tensors: the unchecked render refuses
        layers[0].replace_gaussian_parameters_(mu_raw=layers[0].mu_raw.detach().clone(),
                                               chol_raw=layers[0].chol_raw.detach().clone(),
                                               amp=layers[0].amp.detach().clone())
    with pytest.raises(RuntimeError, match="earlier checked render"):
        fb.render(check=False)


def _densify_clone(layer, idx, noise):
    """The reference's clone (controllers/clone.py:31-56): the selected Gaussians are appended
    with mu_raw + noise, and the originals and the clones each keep half the amplitude."""
    mu, chol, amp = layer.mu_raw.detach(), layer.chol_raw.detach(), layer.amp.detach()
    idx = torch.as_tensor(idx, dtype=torch.long, device=mu.device)
    new_amp = amp.clone()
    new_amp[idx] = new_amp[idx] * 0.5
    layer.replace_gaussian_parameters_(mu_raw=torch.cat([mu, mu.index_select(0, idx) + noise]),
                                       chol_raw=torch.cat([chol, chol.index_select(0, idx)]),
                                       amp=torch.cat([new_amp, amp.index_select(0, idx) * 0.5]))


def _densify_prune(layer, keep):
    """The reference's prune (controllers/prune.py:38-45): rows of the keep mask."""
    keep = keep.to(layer.mu_raw.device)
    layer.replace_gaussian_parameters_(mu_raw=layer.mu_raw.detach()[keep], chol_raw=layer.chol_raw.detach()[keep],
                                       amp=layer.amp.detach()[keep])


@pytest.mark.parametrize("tile", [16, 32])
def test_gaussian_field_batch_densification(device, tile):
    """Densification between training steps (reference base_trainer.py:126-220: clone and prune
    replace a layer's parameters with tensors of another K): GaussianFieldBatch re-plans in
    place and keeps matching per-layer rendering; K changes within k_capacity reuse every
    workspace and the plan buffer, and a layer grown past it gets larger buffers."""
    import copy

    from guass_amd.layers import GaussianAdapterConfig, GaussianFieldBatch, GaussianLinear

    torch.manual_seed(11)
    shapes = [(96, 80, 48), (64, 64, 24), (120, 40, 36)]  # (in, out, K)
    layers_a, layers_b = [], []
    for n_in, n_out, k in shapes:
        cfg = GaussianAdapterConfig(init_num_gaussians=k, tile_out=tile, tile_in=tile, adapter_scale=0.5,
                                    init_amp_scale=1e-2)
        la = GaussianLinear(n_in, n_out, adapter_config=cfg, device=device)
        with torch.no_grad():
            la.chol_raw.add_(torch.randn_like(la.chol_raw) * 0.2)
        layers_a.append(la)
        layers_b.append(copy.deepcopy(la))
    fb = GaussianFieldBatch(layers_b, k_capacity=64)
    xs = [torch.randn(5, n_in, device=device) for (n_in, _, _) in shapes]

    def buffers():
        return [(pl.fwd_ws.data_ptr(), pl.bwd_ws.data_ptr()) for pl in fb._plan.plans], fb._plan.plan.data_ptr()

    g = torch.Generator(device="cpu").manual_seed(5)
    events = [  # (layer, "clone" indices | "prune" keep count) after each step
        [(0, "clone", 6), (1, "prune", 20)],
        [(2, "clone", 10)],
        [(1, "clone", 50)],  # 20 -> 70: past the capacity of 64
        [(0, "prune", 30)],
    ]
    prev = None
    for step in range(len(events) + 1):
        for ls in (layers_a, layers_b):
            for ly in ls:
                for q in (ly.mu_raw, ly.chol_raw, ly.amp):
                    q.grad = None
        ks = [ly.num_gaussians for ly in layers_b]
        say(f"densification step {step}: K={ks} tile {tile}")
        loss_a = sum((ly(x) ** 2).sum() for ly, x in zip(layers_a, xs))
        loss_a.backward()
        fb.render()
        outs_b = [ly(x) for ly, x in zip(layers_b, xs)]
        sum((o ** 2).sum() for o in outs_b).backward()
        torch.cuda.synchronize()
        for i in range(3):
            with torch.no_grad():
                ya = layers_a[i](xs[i])
            assert torch.equal(outs_b[i].detach(), ya), f"step {step} layer {i}: output"
            for name in ("mu_raw", "chol_raw", "amp"):
                grad_close(getattr(layers_b[i], name).grad, getattr(layers_a[i], name).grad,
                           f"step {step} layer {i} {name}", rtol=1e-5)
        now = buffers()
        if prev is not None:
            grown = {i for i, k in enumerate(ks) if k > 64 and prev_ks[i] <= 64}
            for i in range(3):
                if i in grown:
                    assert now[0][i] != prev[0][i], f"step {step} layer {i}: buffers should have grown"
                else:
                    assert now[0][i] == prev[0][i], f"step {step} layer {i}: workspace reallocated"
            if not grown:
                assert now[1] == prev[1], f"step {step}: plan buffer reallocated"
        prev, prev_ks = now, ks
        if step == len(events):
            break
        with torch.no_grad():  # an Adam-sized step (lr * sign), then the same parameters on both copies
            for la, lb in zip(layers_a, layers_b):
                for name in ("mu_raw", "chol_raw", "amp"):
                    pa, pb = getattr(la, name), getattr(lb, name)
                    pa.add_(pa.grad.sign(), alpha=-1e-3)
                    pb.copy_(pa)
        for i, kind, n in events[step]:
            K = layers_a[i].num_gaussians
            if kind == "clone":
                idx = torch.randint(0, K, (n,), generator=g)
                noise = (torch.randn(n, 2, generator=g) * 1e-2).to(device)
                for ls in (layers_a, layers_b):
                    _densify_clone(ls[i], idx, noise)
            else:
                keep = torch.zeros(K, dtype=torch.bool)
                keep[torch.randperm(K, generator=g)[:n]] = True
                for ls in (layers_a, layers_b):
                    _densify_prune(ls[i], keep)
    assert fb.replans >= len(events)


@pytest.mark.parametrize("shape", [(320, 768), (1280, 1792)], ids=["320x768", "1280x1792_stripes8"])
def test_field_plan_resize_within_capacity(device, shape):
    """A single-field FieldPlan moved between K values (densification: clone and prune,
    reference controllers/clone.py:31-56, prune.py:34-45) within its k_capacity: forward and
    backward against the oracle at every K, with no buffer reallocated; past the capacity its
    buffers grow.  The 1280x1792 field (8960 tiles) has eight accumulator stripes, laid out
    stripe-major by the current K, so the backward after each K change reads slots the previous
    K's layout left zeroed."""
    M, N = shape
    plan = FieldPlan(M, N, 64, device, ids_capacity=1 << 18, k_capacity=512)
    bufs = (plan.fwd_ws.data_ptr(), plan.bwd_ws.data_ptr(), plan.ids.data_ptr(), plan._d_mu.data_ptr())
    ks = ((64, 1), (300, 2), (512, 3), (100, 4), (700, 5)) if M == 320 else ((200, 1), (512, 3), (100, 4))
    for k, seed in ks:
        p = wl.make_problem(f"resize_{M}x{N}_k{k}", M, N, k, math.log(6.0), 0.7, seed)
        grew = plan.resize(k)
        say(f"FieldPlan.resize to K={k}: grew={grew}")
        assert grew == (k > 512), f"K={k}: reallocation {grew}"
        if k <= 512:
            assert (plan.fwd_ws.data_ptr(), plan.bwd_ws.data_ptr(), plan.ids.data_ptr(),
                    plan._d_mu.data_ptr()) == bufs
        q = p.to(device)
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        d_mu, d_chol, d_amp = plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        torch.cuda.synchronize()
        assert plan.status() == 0
        r = oracle(p)
        P = int(r[1][-1])
        binning_equal(plan.tile_ptr, plan.ids[:P], r[1], r[2])
        field_close(plan.delta, r[0])
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (d_mu, d_chol, d_amp), r[3:]):
            grad_close(a, b, f"K={k} {name}")
        # the one-launch backward at this K (its maps and gradient slots move with K)
        if plan.direct_launches(P) == 1:
            plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
            direct = plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                          num_pairs=P)
            torch.cuda.synchronize()
            for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), direct, r[3:]):
                grad_close(a, b, f"K={k} {name} (direct)")


def test_graph_replay_direct_backward(device):
    """forward + backward_direct captured in one HIP graph (the bench's step), replayed three
    times with eager work and poisoned outputs between the replays: every replay's delta-W,
    ids and gradients against the eager step (the forward's clearing of the gradient slots is
    a kernel, not a memset)."""
    p = wl.cfg3(7)
    q = p.to(device)
    r = oracle(p)
    P = int(r[1][-1])
    plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P)
    assert plan.direct_launches(P) == 1
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        eager = [t.clone() for t in plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw,
                                                         q.amp, num_pairs=P)]
    torch.cuda.current_stream(device).wait_stream(s)
    torch.cuda.synchronize()
    delta0, ids0 = plan.delta.clone(), plan.ids[:P].clone()
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), eager, r[3:]):
        grad_close(a, b, f"eager {name}")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        views = plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P)
    for rep in range(3):
        plan.delta.fill_(float("nan"))
        for v in views:
            v.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert plan.status() == 0 and plan.status("backward") == 0
        assert torch.equal(plan.delta, delta0), f"replay {rep}: delta"
        assert torch.equal(plan.ids[:P], ids0), f"replay {rep}: ids"
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), views, eager):
            grad_close(a, b, f"replay {rep} {name}", rtol=1e-5)
        _ = (plan.delta * 2.0).sum().item()  # eager work between replays


def run_plan(p: wl.FieldProblem, device, capacity: int, **cfg):
    """The sync-free FieldPlan path: the forward workspace (and its heavy-tile list) reaches the
    backward, as in GaussianFieldCudaTrainFunction."""
    q = p.to(device)
    plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=capacity, **cfg)
    plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    grads = plan.backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    torch.cuda.synchronize()
    P = int(plan.tile_ptr[-1])
    return plan, (plan.delta.clone(), plan.tile_ptr.clone(), plan.ids[:min(P, capacity)].clone(),
                  *(t.clone() for t in grads))


def _clustered_problem(name, M, N, K, seed, clusters, cluster_sigma_px, log_scale_px, n_bad=0):
    p = wl.make_problem(name, M, N, K, log_scale_px, 0.3, seed, clusters=clusters,
                        cluster_sigma_px=cluster_sigma_px)
    if n_bad:
        bad = _indefinite_problem(M, N, seed, n_normal=1, n_bad=n_bad)
        # elongated indefinite Gaussians through the first cluster's heavy tiles
        centre = p.mu[: K // clusters].mean(0)
        p.mu = torch.cat([p.mu, centre + 0.02 * torch.randn(n_bad, 2, generator=torch.Generator().manual_seed(seed))])
        p.chol_raw = torch.cat([p.chol_raw, bad.chol_raw[1:]])
        p.amp = torch.cat([p.amp, bad.amp[1:]])
    return p


def _heavy_tiles(tile_ptr) -> int:
    return int(((tile_ptr[1:] - tile_ptr[:-1]) > HEAVY_TILE).sum())


HEAVY_CASES = {
    # dense (pairs >= 16 per tile: transposing sums), clusters of 2048 Gaussians
    "dense": dict(M=192, N=256, K=2048, clusters=2, cluster_sigma_px=14.0, log_scale_px=math.log(4.0)),
    # sparse (row sums), one tight cluster in a large field
    "sparse": dict(M=640, N=640, K=2048, clusters=1, cluster_sigma_px=10.0, log_scale_px=math.log(2.0)),
    # clamp below 80 (masked moments), normalisation, indefinite Gaussians inside heavy tiles
    "clamp24": dict(M=192, N=256, K=2048, clusters=2, cluster_sigma_px=14.0, log_scale_px=math.log(4.0),
                    cfg=dict(clamp_quad=24.0)),
    "normalize": dict(M=256, N=192, K=2100, clusters=3, cluster_sigma_px=12.0, log_scale_px=math.log(3.0),
                      cfg=dict(normalize=True)),
    "indefinite": dict(M=256, N=192, K=2100, clusters=3, cluster_sigma_px=12.0, log_scale_px=math.log(3.0),
                       n_bad=6),
}


@pytest.mark.parametrize("case", list(HEAVY_CASES))
def test_heavy_tiles_plan(device, case):
    """Tiles of more than HEAVY_TILE Gaussians (k_bin_tiles lists them; the render and backward give each
    a workgroup of four waves) through the sync-free plan, against the oracle: binning bit-exact,
    field and gradients at the parity bars."""
    c = dict(HEAVY_CASES[case])
    cfg = c.pop("cfg", {})
    p = _clustered_problem(f"heavy_{case}", seed=40, **c)
    kw = dict(normalize=cfg.get("normalize", False), clamp=cfg.get("clamp_quad", 80.0))
    say(f"{p.name} M={p.out_features} N={p.in_features} K={p.k} {cfg}")
    r = oracle(p, batched=True, **kw)
    P = int(r[1][-1])
    heavy = _heavy_tiles(r[1])
    say(f"  pairs={P} tiles={r[1].numel() - 1} heavy tiles={heavy}")
    assert heavy > 0
    plan, g = run_plan(p, device, P, **cfg)
    assert plan.status() == 0 and plan.status("backward") == 0
    binning_equal(g[1], g[2], r[1], r[2])
    field_close(g[0], r[0])
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), g[3:], r[3:]):
        grad_close(a, b, name)


def test_heavy_tiles_cfg5c_plan_and_determinism(device):
    """cfg5c (clustered: 271 heavy tiles, up to 151 Gaussians per tile) through the sync-free plan
    against the oracle, and a second forward bit-identical to the first (the heavy tiles' partial
    sums are added in wave order, whichever workgroup takes the tile)."""
    p = wl.cfg5c(0)
    r = oracle(p, batched=True)
    P = int(r[1][-1])
    assert _heavy_tiles(r[1]) > 200
    plan, g = run_plan(p, device, P)
    assert plan.status() == 0
    binning_equal(g[1], g[2], r[1], r[2])
    field_close(g[0], r[0])
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), g[3:], r[3:]):
        grad_close(a, b, name)
    q = p.to(device)
    plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    torch.cuda.synchronize()
    assert torch.equal(plan.delta, g[0]) and torch.equal(plan.ids[:P], g[2])


@pytest.mark.parametrize("case", ["dense", "indefinite"])
def test_heavy_tiles_autograd_train_function(device, case):
    """Heavy tiles through the reference's autograd entry point (runtime.gaussian_field_train,
    runtime.py:273-297): its backward receives the forward workspace kept on ctx, so it takes the
    heavy-tile kernels (the one-launch kernel where the widest rectangle allows it, else the
    reduction + finish); gradients against the oracle."""
    c = dict(HEAVY_CASES[case])
    c.pop("cfg", None)
    p = _clustered_problem(f"heavy_autograd_{case}", seed=42, **c)
    q = p.to(device)
    mu = q.mu.clone().requires_grad_(True)
    raw = q.chol_raw.clone().requires_grad_(True)
    amp = q.amp.clone().requires_grad_(True)
    delta = runtime.gaussian_field_train(row_coords=q.row_coords, col_coords=q.col_coords, mu=mu,
                                         chol_raw=raw, amp=amp, tile_out=16, tile_in=16,
                                         sigma_multiplier=3.0, normalize=False, clamp_quad=80.0)
    (delta * q.grad.view_as(delta)).sum().backward()
    torch.cuda.synchronize()
    r = oracle(p, batched=True)
    assert _heavy_tiles(r[1]) > 0
    field_close(delta, r[0])
    grad_close(mu.grad, r[3], "mu.grad")
    grad_close(raw.grad, r[4], "chol_raw.grad")
    grad_close(amp.grad, r[5], "amp.grad")


def test_one_layer_batch_survives_k_changes(device):
    """A single layer that must keep a captured graph across densification runs as a batch of
    one: a graph captured over forward + backward at K = 200 is replayed after update()
    re-plans the same plan for K = 480 and 90 (k_capacity 512).  No buffer or plan pointer
    changes, and every replay matches the oracle for the current K."""
    from guass_amd.ops import FieldBatchPlan

    p0 = wl.make_problem("one_layer_k200", 320, 768, 200, math.log(6.0), 0.7, 1)
    batch = FieldBatchPlan([p0.to(device)], device, capacities=[1 << 16], k_capacities=[512])
    pl = batch.plans[0]

    def pointers():
        return (pl.fwd_ws.data_ptr(), pl.bwd_ws.data_ptr(), pl.ids.data_ptr(), pl.delta.data_ptr(),
                batch.plan.data_ptr(), batch.grad_flat.data_ptr())

    first = (batch.info.tile_blocks, batch.info.emit_blocks, batch.info.finish_blocks, batch.info.render_blocks, batch.info.tile_render,
             batch.info.plan_bytes)
    ptrs = pointers()
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        batch.forward()
        batch.backward()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            batch.forward()
            batch.backward()
    torch.cuda.current_stream(device).wait_stream(s)
    torch.cuda.synchronize()
    for k, seed in ((200, 1), (480, 2), (90, 3)):
        p = wl.make_problem(f"one_layer_k{k}", 320, 768, k, math.log(6.0), 0.7, seed)
        assert batch.update([p.to(device)]), f"K={k}: re-planned with new grids"
        assert not batch.reallocated and pointers() == ptrs, f"K={k}: a buffer was reallocated"
        assert (batch.info.tile_blocks, batch.info.emit_blocks, batch.info.finish_blocks, batch.info.render_blocks, batch.info.tile_render,
                batch.info.plan_bytes) == first
        pl.delta.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        say(f"  K={k}: graph replayed after the re-plan")
        assert batch.status() == [0]
        r = oracle(p)
        binning_equal(pl.tile_ptr, pl.ids[:int(r[1][-1])], r[1], r[2])
        field_close(pl.delta, r[0])
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), r[3:]):
            grad_close(a, b, f"K={k} {name}")


def test_heavy_tiles_capacity_overflow(device):
    """An id capacity below the pair count on a field with heavy tiles: GF_STATUS_CAPACITY, and
    every kernel returns (the heavy-tile grid is sized from the capacity)."""
    c = dict(HEAVY_CASES["dense"])
    p = _clustered_problem("heavy_overflow", seed=41, **c)
    r = oracle(p, batched=True)
    P = int(r[1][-1])
    plan, _ = run_plan(p, device, P // 3)
    assert plan.status() & _native.GF_STATUS_CAPACITY


@pytest.mark.parametrize("tile", [16, 32])
def test_batch_plan_update_keeps_captured_graph_valid(device, tile):
    """A graph captured over gf_batch_forward + gf_batch_backward before every layer's K and
    parameter tensors change (densification) replays correctly after FieldBatchPlan.update()
    re-plans in place within k_capacity: binning, delta-W and gradients as the single-field
    path gives for the new fields, and no buffer reallocated."""
    from guass_amd.ops import FieldBatchPlan

    before = [wl.cfg1(6), wl.make_problem("cfg2_k256_s7", 320, 768, 256, math.log(6.0), 0.7, 7),
              tiny_problem(80, 96, 40, 8)]
    after = [wl.make_problem("cfg1_k150_s9", 320, 320, 150, math.log(4.0), 0.5, 9),
             wl.make_problem("cfg2_k190_s10", 320, 768, 190, math.log(6.0), 0.7, 10),
             tiny_problem(80, 96, 96, 11)]
    singles = {}
    for name, probs in (("before", before), ("after", after)):
        singles[name] = [run_gpu(p, device, tile_out=tile, tile_in=tile) for p in probs]
    caps = [max(int(a[1][-1]), int(b[1][-1])) for a, b in zip(singles["before"], singles["after"])]
    qa = [p.to(device) for p in before]
    batch = FieldBatchPlan(qa, device, capacities=caps, k_capacities=[256] * 3, tile_out=tile, tile_in=tile)
    bufs = ([(pl.fwd_ws.data_ptr(), pl.bwd_ws.data_ptr(), pl.ids.data_ptr()) for pl in batch.plans],
            batch.plan.data_ptr(), batch.grad_flat.data_ptr())
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        batch.forward()
        batch.backward()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            batch.forward()
            batch.backward()
    torch.cuda.current_stream(device).wait_stream(s)
    torch.cuda.synchronize()

    def verify(name):
        assert batch.status() == [0] * 3, name
        for i, (pl, sg) in enumerate(zip(batch.plans, singles[name])):
            P = int(sg[1][-1])
            assert torch.equal(pl.tile_ptr, sg[1]) and torch.equal(pl.ids[:P], sg[2]), f"{name} {i}: binning"
            assert torch.equal(pl.delta, sg[0]), f"{name} {i}: delta"
            for gname, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), (pl.d_mu, pl.d_chol_raw, pl.d_amp), sg[3:]):
                grad_close(a, b, f"{name} layer {i} {gname}", rtol=1e-5)

    for name, probs in (("before", None), ("after", after)):
        if probs is not None:
            say(f"re-plan in place: K {[p.k for p in before]} -> {[p.k for p in probs]} tile {tile}")
            qb = [p.to(device) for p in probs]
            assert batch.update(qb), "launch grids changed within k_capacity"
            now = ([(pl.fwd_ws.data_ptr(), pl.bwd_ws.data_ptr(), pl.ids.data_ptr()) for pl in batch.plans],
                   batch.plan.data_ptr(), batch.grad_flat.data_ptr())
            assert now == bufs, "a buffer was reallocated within the capacities"
        graph.replay()
        torch.cuda.synchronize()
        verify(name)


def test_adapter_checkpoint_delta_w(device, tmp_path):
    """A trained adapter (a few SGD steps on the GPU) saved in the gaussian-peft-adapter format
    and loaded into a fresh model: its delta-W equals the trained layer's bit for bit and the
    oracle's at the field tolerance (checkpoints/io.py:18-39; scripts/sample_eval_10751.py:231-239
    loads adapters this way for sampling)."""
    from guass_amd.checkpoints import load_adapter_checkpoint, save_adapter_checkpoint
    from guass_amd.layers import GaussianAdapterConfig, GaussianLinear

    torch.manual_seed(3)
    cfg = GaussianAdapterConfig(init_num_gaussians=40, tile_out=16, tile_in=16, init_amp_scale=1e-2)
    model = torch.nn.ModuleDict({"to_k": GaussianLinear(96, 80, adapter_config=cfg, device=device)})
    layer = model["to_k"]
    opt = torch.optim.SGD([layer.mu_raw, layer.chol_raw, layer.amp], lr=1e-3)
    x = torch.randn(8, 96, device=device)
    say("adapter checkpoint: 3 SGD steps, save, load, delta-W")
    before = [t.detach().clone() for t in (layer.mu_raw, layer.chol_raw, layer.amp)]
    for _ in range(3):
        opt.zero_grad()
        (layer(x) ** 2).mean().backward()
        opt.step()
    for b0, t in zip(before, (layer.mu_raw, layer.chol_raw, layer.amp)):
        assert not torch.equal(b0, t.detach())  # trained: every parameter moved
    path = str(tmp_path / "adapter.pt")
    save_adapter_checkpoint(path, model, ["to_k"], cfg, step=3)
    fresh = torch.nn.ModuleDict({"to_k": GaussianLinear(96, 80, adapter_config=cfg, device=device)})
    load_adapter_checkpoint(path, fresh)
    with torch.no_grad():
        want = layer.compute_delta_weight()
        got = fresh["to_k"].compute_delta_weight()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    ly = fresh["to_k"]
    ref = fo.gaussian_field_fwd_bwd(ly.row_coords.cpu(), ly.col_coords.cpu(), ly.materialize_mu().detach().cpu(),
                                    ly.chol_raw.detach().cpu(), ly.amp.detach().cpu(),
                                    torch.zeros(80 * 96), 16, 16, 3.0, False, 80.0)
    field_close(got.reshape(-1), ref[0])


def _indefinite_problem(M: int, N: int, seed: int, n_normal: int = 24, n_bad: int = 6):
    """Ordinary Gaussians plus extremely elongated ones whose fp32 covariance L L^T is no longer
    positive definite after rounding (det < 0: l11, l22 at the softplus floor, |l21| ~ 100).
    The reference's torch path inverts such a matrix exactly; the negative quadratic forms its
    clamp maps to q = 0 give the Gaussian its full amplitude there."""
    p = tiny_problem(M, N, n_normal, seed)
    gen = torch.Generator().manual_seed(seed)
    found = []
    while len(found) < n_bad:
        raw = torch.empty(64, 3)
        raw[:, 0] = -100.0 - 100.0 * torch.rand(64, generator=gen)
        raw[:, 1] = (50.0 + 100.0 * torch.rand(64, generator=gen)) * torch.sign(torch.randn(64, generator=gen))
        raw[:, 2] = -100.0 - 100.0 * torch.rand(64, generator=gen)
        cov = fo.activate_cholesky(raw)
        cov = cov @ cov.transpose(-1, -2)  # fp32, as the reference forms it
        c64 = cov.double()
        det = c64[:, 0, 0] * c64[:, 1, 1] - c64[:, 0, 1] * c64[:, 1, 0]
        found += [raw[i] for i in range(64) if det[i] < 0][: n_bad - len(found)]
    bad = torch.stack(found)
    mu_bad = (torch.rand(n_bad, 2, generator=gen) * 1.6 - 0.8)
    amp_bad = torch.randn(n_bad, 1, generator=gen) * 1e-2
    p.mu = torch.cat([p.mu, mu_bad])
    p.chol_raw = torch.cat([p.chol_raw, bad])
    p.amp = torch.cat([p.amp, amp_bad])
    return p


@pytest.mark.parametrize("tile", [16, 32])
def test_indefinite_fp32_covariances(device, tile):
    p = _indefinite_problem(80, 96, 31 + tile)
    check(p, device, tile_out=tile, tile_in=tile)


def test_delta_apply_merged_matches_row_chunk(device):
    """delta_apply="merged" (one GEMM on W + delta-W) against the reference's row-chunked
    composition (gaussian_linear.py:222-253): outputs and gradients at fp32 GEMM tolerance."""
    import copy

    from guass_amd.layers import GaussianAdapterConfig, GaussianLinear

    torch.manual_seed(11)
    cfg = GaussianAdapterConfig(init_num_gaussians=32, tile_out=16, tile_in=16, init_amp_scale=1e-2,
                                adapter_scale=0.7)
    a = GaussianLinear(96, 200, adapter_config=cfg, device=device)
    b = copy.deepcopy(a)
    b.adapter_config = copy.copy(cfg)
    b.adapter_config.delta_apply = "merged"
    x = torch.randn(3, 7, 96, device=device)
    ya, yb = a(x), b(x)
    (ya.square().sum()).backward()
    (yb.square().sum()).backward()
    torch.cuda.synchronize()
    assert a.last_forward_metadata["linear_composition"] == "base_plus_delta_row_chunk_accumulate"
    assert b.last_forward_metadata["linear_composition"] == "merged_weight"
    ya, yb = ya.detach(), yb.detach()
    assert float((ya - yb).abs().max()) <= 1e-5 * float(ya.abs().max())
    for name in ("mu_raw", "chol_raw", "amp"):
        grad_close(getattr(b, name).grad, getattr(a, name).grad, name, rtol=1e-4)


class _MergedView:
    """A FieldBatchPlan layer (a problem on the device) with a merged consumer."""

    def __init__(self, q, base_weight=None, delta_scale=1.0, keep_delta=True):
        for name in ("row_coords", "col_coords", "mu", "chol_raw", "amp"):
            setattr(self, name, getattr(q, name))
        self.grad = None
        if base_weight is not None:
            self.base_weight, self.delta_scale, self.keep_delta = base_weight, delta_scale, keep_delta


@pytest.mark.parametrize("tile", [16, 32])
def test_batch_merged_weight_matches_torch(device, tile):
    """The batched render's merged output (gf_layer.merged_weight) equals torch's
    `weight + delta * scale` on the same delta-W bit for bit, and the backward given
    dL/d(merged weight) G equals the plain backward given dL/d(delta) = G * scale within 1e-5.
    Layers: cfg2, a ragged 100x77 field (unaligned rows: the scalar store path), and (16x16) a
    layer whose K capacity past the masks renders it tile by tile; delta-W kept or not."""
    from guass_amd.ops import FieldBatchPlan

    probs = [wl.cfg2(3), wl.make_problem("ragged_100x77_k40", 100, 77, 40, math.log(4.0), 0.5, 41)]
    kcaps = [None, None]
    if tile == 16:
        probs.append(wl.cfg1(4))
        kcaps.append(9000)  # capacity on the emission path: k_render16_batch
    qs = [p.to(device) for p in probs]
    gen = torch.Generator(device=device).manual_seed(7)
    ws = [torch.randn(p.out_features, p.in_features, device=device, generator=gen) * 0.02 for p in probs]
    gs = [torch.randn(p.out_features * p.in_features, device=device, generator=gen) for p in probs]
    scale = 0.7
    caps = [int(oracle(p, tile_out=tile, tile_in=tile)[1][-1]) + 64 for p in probs]
    plain_views = [_MergedView(q) for q in qs]
    merged_views = [_MergedView(q, w, scale, keep_delta=(i % 2 == 0)) for i, (q, w) in enumerate(zip(qs, ws))]
    plain = FieldBatchPlan(plain_views, device, capacities=caps, k_capacities=kcaps, tile_out=tile, tile_in=tile)
    merged = FieldBatchPlan(merged_views, device, capacities=caps, k_capacities=kcaps, tile_out=tile, tile_in=tile)
    say(f"merged batch ({tile}x{tile}): {[p.name for p in probs]}, tile_render={merged.info.tile_render}")
    if tile == 16:
        assert merged.info.tile_render == 1 and merged.info.render_blocks > 0
    for v, g in zip(plain_views, gs):
        v.grad = g * scale  # what autograd hands delta-W through `delta * scale`
    for v, g in zip(merged_views, gs):
        v.grad = g
    plain.update()
    merged.update()
    for pl in merged.plans:
        pl.delta.fill_(float("nan"))
    plain.forward()
    merged.forward()
    plain.backward()
    merged.backward()
    torch.cuda.synchronize()
    assert plain.status() == [0] * len(probs) and merged.status() == [0] * len(probs)
    _, _, n_plain = plain.read(norms=True)
    _, _, n_merged = merged.read(norms=True)
    assert n_plain == n_merged
    for i, (a, b, w) in enumerate(zip(plain.plans, merged.plans, ws)):
        d = a.delta.view(a.M, a.N)
        assert torch.equal(merged.merged[i], w + d * scale), f"layer {i}: merged weight"
        assert merged.merged[i].shape == (a.M, a.N) and plain.merged[i] is None
        if i % 2 == 0:
            assert torch.equal(b.delta, a.delta), f"layer {i}: kept delta-W"
        else:
            assert bool(torch.isnan(b.delta).all()), f"layer {i}: delta-W written though not kept"
        for name in ("d_mu", "d_chol_raw", "d_amp"):
            grad_close(getattr(b, name), getattr(a, name), f"layer {i} {name}", rtol=1e-5)


def test_gaussian_field_batch_merged_layers(device):
    """GaussianLinear layers with delta_apply="merged" in a GaussianFieldBatch take weight +
    adapter_scale * delta-W from the batched render: one layer of each SD1.5 attention shape
    (K = 1024).  Outputs and gradients against the same layers rendering their own delta-W and
    composing it in eager torch (gradients within 1e-5), and the gradients against the CPU
    oracle through tanh with dL/d(delta-W) = adapter_scale * dL/d(merged weight)."""
    import copy

    from guass_amd.layers import GaussianFieldBatch

    probs = [_cfg4_layer(i) for i in SD15_SHAPE_PICK]
    scale = 0.5
    batched_layers = _layers_from_problems(probs, device)
    gen = torch.Generator(device=device).manual_seed(9)
    for ly in batched_layers:
        ly.adapter_config.delta_apply = "merged"
        ly.adapter_config.adapter_scale = scale
        with torch.no_grad():
            ly.weight.copy_(torch.randn(ly.weight.shape, device=device, generator=gen) * 0.02)
    eager_layers = [copy.deepcopy(ly) for ly in batched_layers]
    for ly in eager_layers:
        ly.adapter_config = copy.copy(ly.adapter_config)
    xs = [torch.randn(5, p.in_features, device=device, generator=gen) for p in probs]
    gys = [torch.randn(5, p.out_features, device=device, generator=gen) for p in probs]
    fb = GaussianFieldBatch(batched_layers)
    outs = fb.render()
    for ly, o in zip(batched_layers, outs):
        assert ly._batched_delta[2] == "merged_weight" and o.shape == ly.weight.shape
    yb = [ly(x) for ly, x in zip(batched_layers, xs)]
    torch.autograd.backward(yb, gys)
    ye = [ly(x) for ly, x in zip(eager_layers, xs)]
    torch.autograd.backward(ye, gys)
    torch.cuda.synchronize()
    for p, a, b, ya, yq, x, gy in zip(probs, batched_layers, eager_layers, yb, ye, xs, gys):
        say(f"  {p.name} {p.out_features}x{p.in_features}: merged batch vs eager, vs oracle")
        assert a.last_forward_metadata["accumulate_backend"] == "batched_fields"
        assert a.last_forward_metadata["linear_composition"] == "merged_weight"
        assert abs(a.last_forward_metadata["delta_w_norm"] - b.last_forward_metadata["delta_w_norm"]) <= \
            1e-6 * b.last_forward_metadata["delta_w_norm"]
        ya, yq = ya.detach(), yq.detach()
        assert float((ya - yq).abs().max()) <= 1e-5 * float(yq.abs().max()), "layer output"
        for name in ("mu_raw", "chol_raw", "amp"):
            grad_close(getattr(a, name).grad, getattr(b, name).grad, f"{name} vs eager", rtol=1e-5)
        g_delta = (gy.t() @ x) * scale  # dL/d(delta-W) through weight + delta-W * scale
        r = fo.gaussian_linear_fwd_bwd(a.row_coords.cpu(), a.col_coords.cpu(), a.mu_raw.detach().cpu(),
                                       a.chol_raw.detach().cpu(), a.amp.detach().cpu(), g_delta.reshape(-1).cpu(),
                                       16, 16, 3.0, False, 80.0, mu_values=torch.tanh(a.mu_raw.detach()).cpu(),
                                       batched=True)
        for name, got, want in zip(("d_mu_raw", "d_chol_raw", "d_amp"), (a.mu_raw.grad, a.chol_raw.grad, a.amp.grad),
                                   r[3:]):
            grad_close(got, want, f"{name} vs oracle")


def _fused_vs_plan(p, device, cfg_kw, cap, P, label):
    """FieldPlan.fwd_bwd_fused against FieldPlan.forward + backward_direct on the same inputs:
    binning identical, delta-W within 1e-5 of the render's maximum (another summation order and
    the backward's form of the exponent), gradients within 1e-5."""
    q = p.to(device)
    fused = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=cap, **cfg_kw)
    ref = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=cap, **cfg_kw)
    fused.delta.fill_(float("nan"))
    d, grads = fused.fwd_bwd_fused(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, q.grad, num_pairs=P)
    grads = [t.clone() for t in grads]
    ref.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
    want = [t.clone() for t in ref.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                                   num_pairs=P)]
    torch.cuda.synchronize()
    assert fused.status() == 0, f"{label}: forward status {fused.status():#x}"
    assert torch.equal(fused.tile_ptr, ref.tile_ptr) and fused.pairs() == P
    assert torch.equal(fused.ids[:P], ref.ids[:P]), f"{label}: ids"
    fin = torch.isfinite(ref.delta)
    assert torch.equal(torch.isfinite(d), fin), f"{label}: non-finite pattern"
    if bool(fin.any()):
        scale = max(float(ref.delta[fin].abs().max()), 1e-30)
        err = float((d[fin] - ref.delta[fin]).abs().max()) / scale
        assert err <= 1e-5, f"{label}: delta-W {err:.2e} from the render"
    for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), grads, want):
        if bool(torch.isfinite(b).all()):
            grad_close(a, b, f"{label} {name} vs forward + backward_direct", rtol=1e-5)
    return fused, d, grads


@pytest.mark.parametrize("case", ["cfg1", "cfg2", "cfg3", "cfg3_clamp24", "cfg2_normalize", "cfg2_noclamp"])
def test_fused_matches_oracle(device, case):
    """gf_fwd_bwd_fused (binning, then one kernel rendering delta-W and reducing dL/d(delta) with the
    same exponentials) against the CPU oracle: binning bit-exact, delta-W within 1e-5, gradients
    within 1e-4; against forward + backward_direct; then a second call with other parameters on
    the same plan (the binning clears the gradient slots the kernel adds into)."""
    base, _, opt = case.partition("_")
    kw = {"clamp24": dict(clamp_quad=24.0), "normalize": dict(normalize=True), "noclamp": dict(clamp_quad=None),
          "": {}}[opt]
    okw = dict(normalize=kw.get("normalize", False), clamp=kw.get("clamp_quad", 80.0))
    plan = None
    for seed in (21, 22):
        p = getattr(wl, base)(seed)
        r = oracle(p, **okw)
        P = int(r[1][-1])
        say(f"fused {case} seed {seed}: M={p.out_features} N={p.in_features} K={p.k} P={P}")
        q = p.to(device)
        if plan is None:
            plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P + 4096, **kw)
            assert plan.fused_supported()
            _fused_vs_plan(p, device, kw, P + 4096, P, case)
        plan.delta.fill_(float("nan"))
        d, grads = plan.fwd_bwd_fused(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, q.grad)
        torch.cuda.synchronize()
        assert plan.status() == 0
        binning_equal(plan.tile_ptr, plan.ids[:P], r[1], r[2])
        field_close(d, r[0])
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), grads, r[3:]):
            grad_close(a, b, f"fused {name}")


@pytest.mark.parametrize("i", range(24))
def test_fused_random_fields(device, i):
    """gf_fwd_bwd_fused on the seeded random fields of test_gf_forward_random_fields (ragged
    sizes, indefinite covariances, normalisation, clamps 24 / 80 / 200 / none, sigma 1.5..3.5):
    against forward + backward_direct, and delta-W at least as close to the float64 evaluation as
    the fp32 oracle.  Fields the one-pass kernel does not take (dense tiles) run the fallback."""
    p, cfg = _random_forward_problem(i)
    r = fo.gaussian_field_fwd_bwd_batched(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, 16, 16,
                                          cfg["sigma"], cfg["normalize"], cfg["clamp"])
    P = int(r[1][-1])
    kw = dict(sigma_multiplier=cfg["sigma"], normalize=cfg["normalize"], clamp_quad=cfg["clamp"])
    cap = max(P, 1)
    say(f"fused {p.name} P={P} {cfg}")
    fused, d, grads = _fused_vs_plan(p, device, kw, cap, P, p.name)
    say(f"  one pass: {fused.fused_supported()}")
    binning_equal(fused.tile_ptr, fused.ids[:P], r[1], r[2])
    r64 = fo.gaussian_field_fwd_bwd_fp64(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad, 16, 16,
                                         cfg["sigma"], cfg["normalize"], cfg["clamp"])
    finite = torch.isfinite(r64[0])
    assert torch.equal(torch.isfinite(d.cpu()), finite)
    if bool(finite.any()):
        scale = max(float(r64[0][finite].abs().max()), 1e-30)
        err_g = float((d.cpu().double() - r64[0])[finite].abs().max()) / scale
        err_o = float((r[0].double() - r64[0])[finite].abs().max()) / scale
        assert err_g <= err_o + 1e-5, (err_g, err_o)
    for k, (name, a) in enumerate(zip(("d_mu", "d_chol_raw", "d_amp"), grads)):
        c = r64[3 + k]
        if not bool(torch.isfinite(c).all()):
            continue
        cn = float(c.norm())
        if cn > 0.0:
            ed = float((a.cpu().double() - c).norm()) / cn
            eo = float((r[3 + k].double() - c).norm()) / cn
            assert ed <= eo + 1e-4, (name, ed, eo)


def test_fused_graph_replay(device):
    """The fused step (binning + one-pass kernel) captured in a HIP graph and replayed three times
    with eager work and poisoned outputs between the replays: every replay's delta-W, ids and
    gradients equal the eager call's (the binning's clearing of the gradient slots is a kernel)."""
    p = wl.cfg3(8)
    q = p.to(device)
    r = oracle(p)
    P = int(r[1][-1])
    plan = FieldPlan(p.out_features, p.in_features, p.k, device, ids_capacity=P)
    assert plan.fused_supported()
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        d, grads = plan.fwd_bwd_fused(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, q.grad)
        eager = [t.clone() for t in grads]
        delta0 = d.clone()
    torch.cuda.current_stream(device).wait_stream(s)
    torch.cuda.synchronize()
    ids0 = plan.ids[:P].clone()
    field_close(delta0, r[0])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        d, views = plan.fwd_bwd_fused(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, q.grad)
    for rep in range(3):
        say(f"  fused replay {rep}")
        plan.delta.fill_(float("nan"))
        plan.ids.fill_(-1)
        for v in views:
            v.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert plan.status() == 0
        assert torch.equal(plan.delta, delta0), f"replay {rep}: delta"
        assert torch.equal(plan.ids[:P], ids0), f"replay {rep}: ids"
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), views, eager):
            grad_close(a, b, f"replay {rep} {name}", rtol=1e-5)
        _ = (plan.delta * 2.0).sum().item()  # eager work between replays


@pytest.mark.parametrize("variant", ["tile16", "tile32", "tile16_two_launch"])
def test_static_plan_graph_survives_k_changes(device, variant):
    """Capacity mode (gf_forward_kcap + gf_backward_direct_kcap through StaticFieldPlan): forward
    and backward captured once at K = 200 (capacity 512) and replayed after set_params with
    K = 480, 90, 0 and 200 again -- no re-capture -- with poisoned outputs and eager work between
    the replays: every replay's binning bit-exact, delta-W and gradients against the oracle of the
    live field.  tile16_two_launch: an id capacity that makes the tiles dense, so the backward is
    the reduction + finish (the same two launches at every K)."""
    from guass_amd.ops import StaticFieldPlan

    tile = 32 if variant == "tile32" else 16
    M = N = 640
    T = (M // tile) * (N // tile)
    full = wl.make_problem("static_640_k480", M, N, 480, math.log(8.0), 0.6, 51)
    # 8 T - 1 (16x16): sparse, no heavy-tile workgroups: the one-launch backward; 16 T: dense, with
    # heavy-tile workgroups (render and reduction) and the finish; 32x32 tiles have no heavy tiles
    cap = {"tile16": 8 * T - 1, "tile32": 16 * T - 1, "tile16_two_launch": 16 * T}[variant]
    plan = StaticFieldPlan(M, N, 512, device, ids_capacity=cap, tile_out=tile, tile_in=tile)
    assert plan.direct_launches() == (2 if variant.endswith("two_launch") else 1)
    q = full.to(device)
    say(f"static plan {variant}: capacity 512, ids capacity {cap}")

    def sub(k):
        return wl.FieldProblem(f"static_k{k}", M, N, full.row_coords, full.col_coords, full.mu[:k].clone(),
                               full.chol_raw[:k].clone(), full.amp[:k].clone(), full.grad)

    plan.set_params(q.mu[:200], q.chol_raw[:200], q.amp[:200])
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):  # warm-up off the capture
        plan.forward(q.row_coords, q.col_coords)
        plan.backward_direct(q.grad, q.row_coords, q.col_coords)
    torch.cuda.current_stream(device).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.forward(q.row_coords, q.col_coords)
        views = plan.backward_direct(q.grad, q.row_coords, q.col_coords)
    for k in (200, 480, 90, 0, 200):
        say(f"  replay with K = {k}")
        plan.set_params(q.mu[:k], q.chol_raw[:k], q.amp[:k])
        plan.delta.fill_(float("nan"))
        for v in views:
            v.fill_(float("nan"))
        float(torch.randn(1 << 12, device=device).sum())  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert plan.status() == 0 and plan.status("backward") == 0, f"K = {k}: status"
        r = oracle(sub(k), tile_out=tile, tile_in=tile)
        P = int(r[1][-1])
        assert plan.pairs() == P
        binning_equal(plan.tile_ptr, plan.ids[:P], r[1], r[2])
        if k == 0:
            assert P == 0 and float(plan.delta.abs().max()) == 0.0
            continue
        field_close(plan.delta, r[0])
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), views, r[3:]):
            grad_close(a[:k], b, f"K = {k} {name}")
