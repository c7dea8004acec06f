"""Synthetic Gaussian fields for the benchmark configurations.

Gaussians are drawn in pixel space -- mean, per-axis log-scale, rotation, amplitude -- and
mapped once, on the CPU in float64, to the reference API's parameterisation: ``mu`` in the
[-1, 1] coordinates of ``torch.linspace(-1, 1, M)`` (kernels/coords.py:23-34), the
softplus-activated Cholesky ``chol_raw[K,3]`` (kernels/covariance.py:14-26) and ``amp[K,1]``.

Draw order with ``torch.Generator().manual_seed(seed)`` (float64): means, log-scales [K,2],
rotations, amplitudes, then dL/d(delta-W).  Everything is cast to float32 once, so the GPU and
the CPU oracle see the same fp32 tensors.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

CHOLESKY_EPS = 1e-5


@dataclass
class FieldProblem:
    """One layer's inputs on the CPU (float32, contiguous)."""

    name: str
    out_features: int
    in_features: int
    row_coords: torch.Tensor
    col_coords: torch.Tensor
    mu: torch.Tensor
    chol_raw: torch.Tensor
    amp: torch.Tensor
    grad: torch.Tensor | None = None
    meta: dict = field(default_factory=dict)

    @property
    def k(self) -> int:
        return int(self.mu.shape[0])

    def to(self, device) -> "FieldProblem":
        mv = lambda t: None if t is None else t.to(device).contiguous()  # noqa: E731
        return FieldProblem(self.name, self.out_features, self.in_features, mv(self.row_coords),
                            mv(self.col_coords), mv(self.mu), mv(self.chol_raw), mv(self.amp),
                            mv(self.grad), dict(self.meta))


def pixel_to_params(M: int, N: int, mean_px: torch.Tensor, log_scale: torch.Tensor,
                    theta: torch.Tensor, amp: torch.Tensor, eps: float = CHOLESKY_EPS):
    """Map pixel-space Gaussians (float64) to (mu, chol_raw, amp) float32.

    Sigma_px = R(theta) diag(e^{2 s1}, e^{2 s2}) R(theta)^T, scaled by D = diag(2/(M-1), 2/(N-1))
    into coordinate units, then factored as L L^T with L lower triangular and the diagonal
    passed through the inverse of softplus(.) + eps.
    """
    mean_px = mean_px.to(torch.float64)
    sr = 2.0 / max(M - 1, 1)
    sc = 2.0 / max(N - 1, 1)
    mu = torch.stack((mean_px[:, 0] * sr - 1.0, mean_px[:, 1] * sc - 1.0), dim=-1)
    c, s = torch.cos(theta), torch.sin(theta)
    v1, v2 = torch.exp(2.0 * log_scale[:, 0]), torch.exp(2.0 * log_scale[:, 1])
    s00 = c * c * v1 + s * s * v2
    s01 = c * s * (v1 - v2)
    s11 = s * s * v1 + c * c * v2
    s00, s01, s11 = s00 * sr * sr, s01 * sr * sc, s11 * sc * sc
    l11 = torch.sqrt(s00)
    l21 = s01 / l11
    l22 = torch.sqrt(torch.clamp(s11 - l21 * l21, min=0.0))
    inv_sp = lambda y: torch.log(torch.expm1(torch.clamp(y - eps, min=1e-7)))  # noqa: E731
    chol_raw = torch.stack((inv_sp(l11), l21, inv_sp(l22)), dim=-1)
    return (mu.to(torch.float32).contiguous(), chol_raw.to(torch.float32).contiguous(),
            amp.reshape(-1, 1).to(torch.float32).contiguous())


def axes(M: int, N: int) -> tuple[torch.Tensor, torch.Tensor]:
    """CPU ``linspace(-1, 1)`` axes (kernels/coords.py:23-34); copy these to the device."""
    return (torch.linspace(-1.0, 1.0, M, dtype=torch.float32),
            torch.linspace(-1.0, 1.0, N, dtype=torch.float32))


def make_problem(name: str, M: int, N: int, K: int, log_scale_mean: float, log_scale_std: float,
                 seed: int, *, clusters: int = 0, cluster_sigma_px: float = 40.0,
                 student_t_scale: float | None = None, amp_std: float = 1e-3,
                 clip_log_scale: float | None = None, with_grad: bool = True) -> FieldProblem:
    g = torch.Generator().manual_seed(seed)
    f64 = torch.float64
    if clusters > 0:
        centres = torch.rand(clusters, 2, generator=g, dtype=f64) * torch.tensor([M, N], dtype=f64)
        pick = torch.randint(0, clusters, (K,), generator=g)
        mean_px = centres[pick] + cluster_sigma_px * torch.randn(K, 2, generator=g, dtype=f64)
        mean_px[:, 0].clamp_(0.0, M - 1.0)
        mean_px[:, 1].clamp_(0.0, N - 1.0)
    else:
        mean_px = torch.rand(K, 2, generator=g, dtype=f64) * torch.tensor([M, N], dtype=f64)
    if student_t_scale is not None:
        z = torch.randn(K, 2, generator=g, dtype=f64)
        chi2 = (torch.randn(K, 2, 3, generator=g, dtype=f64) ** 2).sum(-1)
        log_scale = log_scale_mean + student_t_scale * z / torch.sqrt(chi2 / 3.0)
    else:
        log_scale = log_scale_mean + log_scale_std * torch.randn(K, 2, generator=g, dtype=f64)
    if clip_log_scale is not None:
        log_scale = log_scale.clamp(log_scale_mean - clip_log_scale, log_scale_mean + clip_log_scale)
    theta = torch.rand(K, generator=g, dtype=f64) * math.pi
    amp = amp_std * torch.randn(K, generator=g, dtype=f64)
    mu, chol_raw, amp32 = pixel_to_params(M, N, mean_px, log_scale, theta, amp)
    grad = (torch.randn(M * N, generator=g, dtype=f64).to(torch.float32) if with_grad else None)
    rc, cc = axes(M, N)
    return FieldProblem(name, M, N, rc, cc, mu, chol_raw, amp32, grad,
                        {"seed": seed, "log_scale_mean": log_scale_mean})


# BASELINE.json configs.  cfg1..cfg3 and cfg5 are single layers; cfg4 is a list of layers.
def cfg1(seed: int = 0, **kw) -> FieldProblem:
    return make_problem("cfg1_320x320_k64", 320, 320, 64, math.log(4.0), 0.5, seed, **kw)


def cfg2(seed: int = 0, **kw) -> FieldProblem:
    return make_problem("cfg2_320x768_k256", 320, 768, 256, math.log(6.0), 0.7, seed, **kw)


def cfg3(seed: int = 0, **kw) -> FieldProblem:
    return make_problem("cfg3_1280x1280_k1024", 1280, 1280, 1024, math.log(8.0), 0.6, seed, **kw)


def cfg5(seed: int = 0, t_scale: float = 0.5, **kw) -> FieldProblem:
    return make_problem(f"cfg5_1280x5120_k4096_t{t_scale:g}", 1280, 5120, 4096, math.log(5.0), 0.0,
                        seed, clusters=8, student_t_scale=t_scale, **kw)


def cfg5c(seed: int = 0, **kw) -> FieldProblem:
    """cfg5 with the Student-t log-scales clipped to log 5 +- 1.5 (covariance condition number
    <= e^6 ~ 403): the same size, clustering and load imbalance without the near-degenerate
    Gaussians whose fp32 field is ill-conditioned (see cfg5)."""
    return make_problem("cfg5c_1280x5120_k4096_clip1.5", 1280, 5120, 4096, math.log(5.0), 0.0, seed,
                        clusters=8, student_t_scale=0.5, clip_log_scale=1.5, **kw)


def sd15_attention_shapes() -> list[tuple[str, int, int]]:
    """(name, out_features, in_features) of the 128 attention linears of an SD1.5 UNet.

    16 transformer blocks (widths 320 x5, 640 x5, 1280 x6 incl. the mid block); per block
    attn1 to_q/to_k/to_v/to_out [C,C], attn2 to_q/to_out [C,C] and to_k/to_v [C,768].
    """
    widths = [320] * 2 + [640] * 2 + [1280] * 2 + [1280] + [1280] * 3 + [640] * 3 + [320] * 3
    shapes = []
    for b, c in enumerate(widths):
        for attn in ("attn1", "attn2"):
            for proj in ("to_q", "to_k", "to_v", "to_out"):
                n_in = 768 if (attn == "attn2" and proj in ("to_k", "to_v")) else c
                shapes.append((f"block{b}.{attn}.{proj}", c, n_in))
    return shapes


def cfg4(seed: int = 0, layers: int | None = None, **kw) -> list[FieldProblem]:
    shapes = sd15_attention_shapes()
    if layers is not None:
        shapes = shapes[:layers]
    return [make_problem(f"cfg4_{name}", m, n, 1024, math.log(8.0), 0.6, seed * 1000 + i, **kw)
            for i, (name, m, n) in enumerate(shapes)]


def cfg5s(seed: int = 0, **kw) -> FieldProblem:
    """cfg5's stress variant: Student-t log-scale scale 1.0 instead of 0.5 (1.67M pairs, 65 a
    tile on average, up to 255)."""
    return cfg5(seed, t_scale=1.0, **kw)


CONFIGS = {"cfg1": cfg1, "cfg2": cfg2, "cfg3": cfg3, "cfg5": cfg5, "cfg5c": cfg5c, "cfg5s": cfg5s}
