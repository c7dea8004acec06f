"""GaussianLinear's field path (reference gaussian_linear.py:162-253) without a GPU: config
validation, initialisation and the reference's error on non-CUDA tensors."""

from __future__ import annotations

import pytest
import torch

from guass_amd.layers import GaussianAdapterConfig, GaussianLinear


def test_config_validation_and_aliases():
    cfg = GaussianAdapterConfig(execution_mode="cuda_field_stage3_custom")
    cfg.validate()
    assert cfg.execution_mode == "cuda_field_train"
    for bad in (dict(execution_mode="dense_reference"), dict(tile_out=0), dict(sigma_multiplier=0.0),
                dict(init_num_gaussians=0), dict(merge_weights=True), dict(eps=0.0)):
        with pytest.raises(ValueError):
            GaussianAdapterConfig(**bad).validate()
    with pytest.raises(NotImplementedError):
        GaussianLinear(8, 8, adapter_config=GaussianAdapterConfig(init_method="grid_overlap"))


def test_layer_parameters_and_cpu_error():
    torch.manual_seed(0)
    cfg = GaussianAdapterConfig(init_num_gaussians=10, init_method="uniform_grid")
    layer = GaussianLinear(24, 16, adapter_config=cfg)
    assert layer.num_gaussians == 10 and layer.chol_raw.shape == (10, 3) and layer.amp.shape == (10, 1)
    assert not layer.weight.requires_grad and not layer.bias.requires_grad
    mu = layer.materialize_mu().detach()
    assert float(mu.abs().max()) <= 1.0 and torch.allclose(mu[0], torch.tensor([-1.0, -1.0]), atol=1e-5)
    state = layer.get_adapter_state()
    layer.load_adapter_state({k: v + 0.0 for k, v in state.items()})
    assert torch.equal(layer.amp, state["amp"])
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        layer.compute_delta_weight()


def test_field_batch_checks_layer_configs():
    """GaussianFieldBatch needs 16x16 tiles and one sigma / normalisation for all layers; the
    checks run before any device work."""
    from guass_amd.layers import GaussianFieldBatch

    ok = GaussianAdapterConfig(init_num_gaussians=4, tile_out=16, tile_in=16)
    a = GaussianLinear(32, 32, adapter_config=ok)
    with pytest.raises(ValueError, match="16x16 or 32x32"):
        GaussianFieldBatch([a, GaussianLinear(32, 32, adapter_config=GaussianAdapterConfig(
            init_num_gaussians=4, tile_out=8, tile_in=8))])
    with pytest.raises(ValueError, match="tile shape"):  # 32x32 next to 16x16
        GaussianFieldBatch([a, GaussianLinear(32, 32, adapter_config=GaussianAdapterConfig(init_num_gaussians=4))])
    other = GaussianAdapterConfig(init_num_gaussians=4, tile_out=16, tile_in=16, sigma_multiplier=2.5)
    with pytest.raises(ValueError, match="sigma_multiplier"):
        GaussianFieldBatch([a, GaussianLinear(32, 32, adapter_config=other)])
    with pytest.raises(ValueError, match="at least one"):
        GaussianFieldBatch([])
    with pytest.raises(TypeError):
        GaussianFieldBatch([torch.nn.Linear(4, 4)])


@pytest.mark.parametrize("k", [8, 32, 128, 512])
def test_init_chol_raw_matches_reference_arithmetic(k):
    """Initial chol_raw diagonal = log(expm1(target - eps)) evaluated by torch in the parameter
    dtype (reference gaussian_linear.py:115-125,286-288).  For these K the float64 value rounded
    once to fp32 is an ulp away, so the check tells the two evaluations apart."""
    import math

    cfg = GaussianAdapterConfig(init_num_gaussians=k, init_method="uniform_grid")
    layer = GaussianLinear(16, 16, adapter_config=cfg)
    scale = max(2.0 / math.sqrt(k) * cfg.init_chol_scale_multiplier, cfg.min_cov_diag ** 0.5)
    fp32 = torch.log(torch.expm1(torch.full((k,), scale, dtype=torch.float32) - cfg.eps))
    f64_rounded = torch.full((k,), math.log(math.expm1(scale - cfg.eps)), dtype=torch.float32)
    assert not torch.equal(fp32, f64_rounded)
    raw = layer.chol_raw.detach()
    assert torch.equal(raw[:, 0], fp32) and torch.equal(raw[:, 2], fp32)
    assert float(raw[:, 1].abs().max()) == 0.0
