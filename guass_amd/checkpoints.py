"""Adapter checkpoints in the reference's ``gaussian-peft-adapter`` format, for GaussianLinear
layers on the MI355X runtime (reference gaussian_peft/checkpoints/io.py:18-39 and
state_dict.py:12-90).

The payload is a plain dict saved with ``torch.save``::

    {"format": "gaussian-peft-adapter", "step": int | None,
     "metadata": {"target_modules": [...], "adapter_config": {...}, "gaussian_modules": [...]},
     "adapters": {module_name: {"mu_raw", "chol_raw", "amp": Tensor,
                                "num_gaussians", "in_features", "out_features": int,
                                "has_bias": bool}}}

so checkpoints written by the reference load here and the other way round.  Loading uses
``torch.load(..., weights_only=True)``: the payload holds tensors, dicts, lists and primitives
only, and nothing in the file is executed.  A module's Gaussian count may differ from the
checkpoint's (densified adapters): its parameters are replaced by the checkpoint's.
"""

from __future__ import annotations

from dataclasses import asdict, is_dataclass
from pathlib import Path
from typing import Any

import torch
from torch import Tensor, nn

from guass_amd.layers import GaussianAdapterConfig, GaussianLinear

ADAPTER_FORMAT = "gaussian-peft-adapter"


def gaussian_adapter_state_dict(model: nn.Module) -> dict[str, Any]:
    """Per GaussianLinear module of ``model``: its Gaussian parameters (on the CPU) and shape
    schema (state_dict.py:12-26)."""
    state: dict[str, Any] = {}
    for name, module in model.named_modules():
        if isinstance(module, GaussianLinear):
            state[name] = {
                "mu_raw": module.mu_raw.detach().cpu(),
                "chol_raw": module.chol_raw.detach().cpu(),
                "amp": module.amp.detach().cpu(),
                "num_gaussians": module.num_gaussians,
                "in_features": module.in_features,
                "out_features": module.out_features,
                "has_bias": module.bias is not None,
            }
    return state


def export_adapter_metadata(model: nn.Module, target_modules: list[str],
                            config: GaussianAdapterConfig) -> dict[str, Any]:
    """The checkpoint's metadata block (state_dict.py:47-62): the adapter config as primitives
    (compute_dtype as its string) and the names of the GaussianLinear modules."""
    cfg = asdict(config) if is_dataclass(config) else dict(config)
    cfg["compute_dtype"] = str(config.compute_dtype)
    return {
        "target_modules": list(target_modules),
        "adapter_config": cfg,
        "gaussian_modules": [n for n, m in model.named_modules() if isinstance(m, GaussianLinear)],
    }


def load_gaussian_adapter_state_dict(model: nn.Module, state_dict: dict[str, Any]) -> None:
    """Loads every entry of an adapter state into the GaussianLinear module of the same name
    (state_dict.py:29-44), after checking its shape schema."""
    modules = dict(model.named_modules())
    for name, entry in state_dict.items():
        if name not in modules:
            raise KeyError(f"Gaussian adapter target module {name!r} not found in model")
        module = modules[name]
        if not isinstance(module, GaussianLinear):
            raise TypeError(f"Module {name!r} is not a GaussianLinear")
        _validate_module_schema(name, module, entry)
        module.load_adapter_state({"mu_raw": _as_tensor(entry["mu_raw"]),
                                   "chol_raw": _as_tensor(entry["chol_raw"]),
                                   "amp": _as_tensor(entry["amp"])})


def save_adapter_checkpoint(path: str, model: nn.Module, target_modules: list[str],
                            config: GaussianAdapterConfig, step: int | None = None) -> None:
    """Writes the ``gaussian-peft-adapter`` payload of ``model`` (io.py:18-32)."""
    payload = {
        "format": ADAPTER_FORMAT,
        "step": step,
        "metadata": export_adapter_metadata(model, target_modules, config),
        "adapters": gaussian_adapter_state_dict(model),
    }
    Path(path).parent.mkdir(parents=True, exist_ok=True)
    torch.save(payload, path)


def load_adapter_checkpoint(path: str, model: nn.Module) -> dict[str, Any]:
    """Reads an adapter checkpoint and loads its adapters into ``model`` (io.py:35-39); returns
    the payload."""
    payload = torch.load(path, map_location="cpu", weights_only=True)
    load_gaussian_adapter_state_dict(model, payload.get("adapters", {}))
    return payload


def _validate_module_schema(name: str, module: GaussianLinear, entry: dict[str, Any]) -> None:
    expected = {"in_features": module.in_features, "out_features": module.out_features,
                "has_bias": module.bias is not None}
    actual = {"in_features": entry["in_features"], "out_features": entry["out_features"],
              "has_bias": entry["has_bias"]}
    if expected != actual:
        raise ValueError(f"Adapter schema mismatch for {name!r}: expected {expected}, got {actual}")


def _as_tensor(value: Tensor | Any) -> Tensor:
    if isinstance(value, Tensor):
        return value
    raise TypeError(f"Expected Tensor, got {type(value)!r}")
