"""Adapter checkpoints in the reference's gaussian-peft-adapter format
(gaussian_peft/checkpoints/io.py:18-39, state_dict.py:12-90), without a GPU."""

from __future__ import annotations

import pickle

import pytest
import torch
from torch import nn

from guass_amd.checkpoints import (
    ADAPTER_FORMAT,
    gaussian_adapter_state_dict,
    load_adapter_checkpoint,
    load_gaussian_adapter_state_dict,
    save_adapter_checkpoint,
)
from guass_amd.layers import GaussianAdapterConfig, GaussianLinear


def _model(k: int) -> nn.Module:
    cfg = GaussianAdapterConfig(init_num_gaussians=k, init_amp_scale=1e-2)
    return nn.ModuleDict({
        "proj": GaussianLinear(24, 16, adapter_config=cfg),
        "block": nn.Sequential(nn.ReLU(), GaussianLinear(32, 8, bias=False, adapter_config=cfg)),
        "plain": nn.Linear(4, 4),
    })


def test_round_trip_and_payload_layout(tmp_path):
    torch.manual_seed(0)
    src = _model(12)
    cfg = src["proj"].adapter_config
    path = tmp_path / "ckpt" / "adapter.pt"
    save_adapter_checkpoint(str(path), src, ["proj", "block.1"], cfg, step=7)
    dst = _model(5)  # other Gaussian counts: the checkpoint's replace them
    payload = load_adapter_checkpoint(str(path), dst)
    assert payload["format"] == ADAPTER_FORMAT and payload["step"] == 7
    meta = payload["metadata"]
    assert meta["target_modules"] == ["proj", "block.1"]
    assert meta["gaussian_modules"] == ["proj", "block.1"]
    assert meta["adapter_config"]["compute_dtype"] == "torch.float32"
    assert meta["adapter_config"]["init_num_gaussians"] == 12
    assert set(payload["adapters"]) == {"proj", "block.1"}
    entry = payload["adapters"]["block.1"]
    assert entry["num_gaussians"] == 12 and entry["in_features"] == 32 and entry["out_features"] == 8
    assert entry["has_bias"] is False
    for name in ("proj", "block.1"):
        a = dict(src.named_modules())[name]
        b = dict(dst.named_modules())[name]
        assert b.num_gaussians == 12
        for p in ("mu_raw", "chol_raw", "amp"):
            assert torch.equal(getattr(a, p), getattr(b, p))
            assert isinstance(getattr(b, p), nn.Parameter)


def test_reference_layout_payload_loads(tmp_path):
    """A payload written field by field as the reference's save_adapter_checkpoint lays it out."""
    torch.manual_seed(1)
    mu_raw, chol_raw, amp = torch.randn(9, 2), torch.randn(9, 3), torch.randn(9, 1) * 1e-3
    payload = {
        "format": "gaussian-peft-adapter",
        "step": None,
        "metadata": {"target_modules": ["proj"], "adapter_config": {"init_num_gaussians": 9,
                                                                    "compute_dtype": "torch.float32"},
                     "gaussian_modules": ["proj"]},
        "adapters": {"proj": {"mu_raw": mu_raw, "chol_raw": chol_raw, "amp": amp, "num_gaussians": 9,
                              "in_features": 24, "out_features": 16, "has_bias": True}},
    }
    path = tmp_path / "ref_layout.pt"
    torch.save(payload, path)
    model = _model(4)
    load_adapter_checkpoint(str(path), model)
    assert torch.equal(model["proj"].mu_raw, mu_raw) and torch.equal(model["proj"].amp, amp)
    assert model["block"][1].num_gaussians == 4  # not in the checkpoint: untouched


def test_schema_and_lookup_errors():
    model = _model(3)
    state = gaussian_adapter_state_dict(model)
    bad = {"proj": dict(state["proj"], in_features=25)}
    with pytest.raises(ValueError, match="Adapter schema mismatch for 'proj'"):
        load_gaussian_adapter_state_dict(model, bad)
    with pytest.raises(KeyError, match="not found in model"):
        load_gaussian_adapter_state_dict(model, {"missing": state["proj"]})
    with pytest.raises(TypeError, match="is not a GaussianLinear"):
        load_gaussian_adapter_state_dict(model, {"plain": state["proj"]})
    with pytest.raises(TypeError, match="Expected Tensor"):
        load_gaussian_adapter_state_dict(model, {"proj": dict(state["proj"], amp=[0.0, 1.0, 2.0])})


class _NotData:
    def __reduce__(self):
        return (print, ("a pickled callable",))


def test_loader_executes_nothing_from_the_file(tmp_path):
    path = tmp_path / "hostile.pt"
    torch.save({"format": ADAPTER_FORMAT, "adapters": {}, "extra": _NotData()}, path)
    with pytest.raises(pickle.UnpicklingError):
        load_adapter_checkpoint(str(path), _model(2))
