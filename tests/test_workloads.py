"""Synthetic workloads: shapes and parameterisation of the BASELINE configurations (CPU)."""

from __future__ import annotations

import math

import torch

from guass_amd import workloads as wl
from oracle import field_oracle as fo


def test_sd15_attention_shapes():
    shapes = wl.sd15_attention_shapes()
    assert len(shapes) == 128
    assert sum(m * n for _, m, n in shapes) == 93_511_680
    assert sum(1 for _, m, n in shapes if n == 768) == 32  # attn2 to_k / to_v
    assert {m for _, m, _ in shapes} == {320, 640, 1280}


def test_config_shapes_and_draw_order():
    for name, (M, N, K) in {"cfg1": (320, 320, 64), "cfg2": (320, 768, 256),
                            "cfg3": (1280, 1280, 1024), "cfg5": (1280, 5120, 4096),
                            "cfg5c": (1280, 5120, 4096)}.items():
        p = wl.CONFIGS[name](0)
        assert (p.out_features, p.in_features, p.k) == (M, N, K)
        assert p.mu.dtype == p.chol_raw.dtype == p.amp.dtype == p.grad.dtype == torch.float32
        assert p.grad.shape == (M * N,)
        assert torch.equal(p.row_coords, torch.linspace(-1.0, 1.0, M))
    a, b = wl.cfg2(3), wl.cfg2(3)
    assert torch.equal(a.mu, b.mu) and torch.equal(a.grad, b.grad)
    assert not torch.equal(wl.cfg2(4).mu, a.mu)
    layers = wl.cfg4(0, layers=3)
    assert [(p.out_features, p.in_features, p.k) for p in layers] == [(320, 320, 1024)] * 3


def test_pixel_to_params_round_trip():
    """chol_raw activates to a factor whose covariance is the pixel-space one mapped to the
    [-1, 1] coordinates; means map to the coordinates of their pixels."""
    M, N, K = 200, 300, 64
    g = torch.Generator().manual_seed(3)
    f64 = torch.float64
    mean_px = torch.rand(K, 2, generator=g, dtype=f64) * torch.tensor([M - 1, N - 1], dtype=f64)
    log_scale = math.log(5.0) + 0.5 * torch.randn(K, 2, generator=g, dtype=f64)
    theta = torch.rand(K, generator=g, dtype=f64) * math.pi
    amp = torch.randn(K, generator=g, dtype=f64)
    mu, raw, amp32 = wl.pixel_to_params(M, N, mean_px, log_scale, theta, amp)
    sr, sc = 2.0 / (M - 1), 2.0 / (N - 1)
    assert torch.allclose(mu.double(), torch.stack((mean_px[:, 0] * sr - 1, mean_px[:, 1] * sc - 1), 1),
                          atol=1e-6)
    L = fo.activate_cholesky(raw.double(), eps=fo.CHOLESKY_EPS)
    cov = L @ L.transpose(-1, -2)
    c, s = torch.cos(theta), torch.sin(theta)
    v1, v2 = torch.exp(2 * log_scale[:, 0]), torch.exp(2 * log_scale[:, 1])
    want = torch.stack((torch.stack((c * c * v1 + s * s * v2, c * s * (v1 - v2)), -1),
                        torch.stack((c * s * (v1 - v2), s * s * v1 + c * c * v2), -1)), -2)
    D = torch.diag(torch.tensor([sr, sc], dtype=f64))
    want = D @ want @ D
    assert torch.allclose(cov, want, rtol=2e-5, atol=1e-12)
    assert torch.equal(amp32.reshape(-1), amp.to(torch.float32))
