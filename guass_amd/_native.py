"""ctypes binding of ``libgaussfield.so`` (C ABI declared in ``include/gaussfield.h``).

``torch`` is imported before the library is opened: torch ships its own HIP runtime under the
same SONAME (libamdhip64.so.7), so the dynamic loader then binds this library to that runtime
and the process keeps a single HIP runtime.  There is no CPU fallback: if the library is
missing or a call fails, a ``RuntimeError`` is raised.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_uint64, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must precede the dlopen below)

# GUASS_AMD_LIB names another build of the library (e.g. the host-sanitized one the CPU tests run)
LIB_PATH = Path(os.environ.get("GUASS_AMD_LIB") or Path(__file__).resolve().with_name("libgaussfield.so"))

GF_OK = 0
GF_STATUS_CAPACITY = 0x1
GF_STATUS_COUNT_MISMATCH = 0x2
GF_STATUS_TILE_PTR_LAST = 0x4
GF_STATUS_TILE_PTR_ORDER = 0x8
GF_STATUS_IDS_NEGATIVE = 0x10
GF_STATUS_IDS_RANGE = 0x20

# Symbols include/gaussfield.h declares.
EXPORTED = (
    "gf_version", "gf_last_error", "gf_tile_grid", "gf_forward_workspace_bytes",
    "gf_forward_workspace_bytes_max", "gf_backward_workspace_bytes", "gf_forward_bin", "gf_forward_emit", "gf_forward_render",
    "gf_backward", "gf_backward_reduce", "gf_backward_finish", "gf_read_status",
    "gf_selftest_softplus", "gf_batch_plan", "gf_batch_forward", "gf_batch_backward",
    "gf_batch_set_grads", "gf_batch_read", "gf_backward_noalloc", "gf_forward", "gf_backward_direct",
    "gf_forward_grads_offset", "gf_backward_direct_launches", "gf_fwd_bwd_fused", "gf_fwd_bwd_fused_supported",
    "gf_forward_kcap", "gf_backward_direct_kcap", "gf_forward_bin_info", "gf_read_bin_info", "gf_backward_train",
)

GF_PHASE_BIN, GF_PHASE_EMIT, GF_PHASE_RENDER = 0x1, 0x2, 0x4
GF_PHASE_REDUCE, GF_PHASE_FINISH = 0x1, 0x2
GF_PHASE_ALL = 0xFF


class GfFieldConfig(ctypes.Structure):
    """``gf_field_config`` (mirrors the reference ForwardConfig, csrc/field.h:11-18)."""

    _fields_ = [
        ("tile_out", c_int64),
        ("tile_in", c_int64),
        ("sigma_multiplier", c_double),
        ("normalize", c_int32),
        ("has_clamp_quad", c_int32),
        ("clamp_quad", c_double),
    ]


class GfLayer(ctypes.Structure):
    """``gf_layer``: one field of a batch (device pointers)."""

    _fields_ = [
        ("out_features", c_int64), ("in_features", c_int64), ("k", c_int64),
        ("row_coords", c_void_p), ("col_coords", c_void_p), ("mu", c_void_p),
        ("chol_raw", c_void_p), ("amp", c_void_p), ("delta", c_void_p), ("tile_ptr", c_void_p),
        ("num_pairs", c_void_p), ("gaussian_ids", c_void_p), ("ids_capacity", c_int64), ("forward_workspace", c_void_p),
        ("forward_workspace_bytes", c_size_t), ("grad_delta", c_void_p), ("d_mu", c_void_p),
        ("d_chol_raw", c_void_p), ("d_amp", c_void_p), ("backward_workspace", c_void_p),
        ("backward_workspace_bytes", c_size_t), ("k_capacity", c_int64), ("mu_tanh", c_int32),
        ("reserved", c_int32), ("base_weight", c_void_p), ("merged_weight", c_void_p), ("delta_scale", c_float),
        ("reserved2", c_int32),
    ]


class GfBinInfo(ctypes.Structure):
    """``gf_bin_info``: P and the most tiles one Gaussian's rectangle covers."""

    _fields_ = [("num_pairs", c_int64), ("max_span", c_int64)]


class GfBatchInfo(ctypes.Structure):
    """``gf_batch_info``."""

    _fields_ = [
        ("n_layers", c_int32), ("has_backward", c_int32), ("tile_blocks", c_int64),
        ("emit_blocks", c_int64), ("finish_blocks", c_int64), ("plan_bytes", c_size_t),
        ("backward_buffers", c_int32), ("mask_clamp", c_int32), ("render_blocks", c_int64),
        ("tile_render", c_int32), ("reserved", c_int32),
    ]


def make_config(tile_out: int, tile_in: int, sigma_multiplier: float, normalize: bool,
                clamp_quad: float | None) -> GfFieldConfig:
    return GfFieldConfig(int(tile_out), int(tile_in), float(sigma_multiplier), 1 if normalize else 0,
                         0 if clamp_quad is None else 1, 0.0 if clamp_quad is None else float(clamp_quad))


_LIB = None
_P = c_void_p
_CFG = POINTER(GfFieldConfig)


def lib() -> ctypes.CDLL:
    """The loaded library (opened once per process)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m guass_amd.build` (hipcc, gfx950). "
            "There is no CPU fallback for the Gaussian-field kernels.")
    L = ctypes.CDLL(str(LIB_PATH))
    L.gf_version.restype = c_char_p
    L.gf_last_error.restype = c_char_p
    L.gf_tile_grid.argtypes = [c_int64, c_int64, _CFG, POINTER(c_int64), POINTER(c_int64)]
    L.gf_forward_workspace_bytes.argtypes = [c_int64, c_int64, c_int64, _CFG]
    L.gf_forward_workspace_bytes.restype = c_size_t
    L.gf_forward_workspace_bytes_max.argtypes = [c_int64, c_int64, c_int64, _CFG]
    L.gf_forward_workspace_bytes_max.restype = c_size_t
    L.gf_backward_workspace_bytes.argtypes = [c_int64, c_int64, c_int64, _CFG]
    L.gf_backward_workspace_bytes.restype = c_size_t
    L.gf_forward_bin.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, c_size_t, _P]
    L.gf_forward_emit.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, c_int64, _P,
                                  c_size_t, _P]
    L.gf_forward_render.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P,
                                    c_int64, _P, _P, c_size_t, _P]
    L.gf_forward.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, _P, _P,
                             c_size_t, _P]
    L.gf_backward.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, c_int32,
                              _P, c_int32, c_int64, _P, _P, _P, _P, _P, c_size_t, _P]
    L.gf_backward_reduce.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int32,
                                     _P, c_int32, c_int64, _P, _P, c_size_t, _P]
    L.gf_backward_finish.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, c_size_t, _P]
    L.gf_backward_noalloc.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, c_int32,
                                      _P, c_int32, c_int64, _P, _P, _P, _P, _P]
    L.gf_backward_direct.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, c_int64,
                                     c_int64, _P, c_size_t, _P, c_size_t, _P]
    L.gf_forward_bin_info.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, POINTER(GfBinInfo), _P,
                                      c_size_t, _P]
    L.gf_read_bin_info.argtypes = [_P, POINTER(GfBinInfo), _P]
    L.gf_backward_train.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, c_int32, _P, c_int32,
                                    c_int64, c_int64, _P, _P, _P, _P, _P, c_size_t, _P]
    L.gf_forward_grads_offset.argtypes = [c_int64, c_int64, c_int64, _CFG]
    L.gf_forward_grads_offset.restype = c_size_t
    L.gf_backward_direct_launches.argtypes = [_CFG, c_int64, c_int64, c_int64, c_int64, c_int64]
    L.gf_backward_direct_launches.restype = c_int
    L.gf_fwd_bwd_fused.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, _P,
                                   _P, c_size_t, _P]
    L.gf_fwd_bwd_fused_supported.argtypes = [_CFG, c_int64, c_int64, c_int64, c_int64, c_int64]
    L.gf_forward_kcap.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, _P, _P,
                                  c_size_t, _P]
    L.gf_backward_direct_kcap.argtypes = [_CFG, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                          c_int64, _P, c_size_t, _P, c_size_t, _P]
    L.gf_fwd_bwd_fused_supported.restype = c_int
    L.gf_read_status.argtypes = [_P, c_int32, POINTER(c_uint32), _P]
    L.gf_batch_plan.argtypes = [_CFG, POINTER(GfLayer), c_int32, _P, c_size_t, POINTER(GfBatchInfo), _P]
    L.gf_batch_forward.argtypes = [_P, POINTER(GfBatchInfo), c_uint32, _P]
    L.gf_batch_backward.argtypes = [_P, POINTER(GfBatchInfo), c_uint32, _P]
    L.gf_batch_set_grads.argtypes = [_P, POINTER(GfBatchInfo), POINTER(c_void_p), _P]
    L.gf_batch_read.argtypes = [_P, POINTER(GfBatchInfo), c_int32, POINTER(c_uint32), POINTER(c_int64),
                                POINTER(c_double), _P]
    L.gf_selftest_softplus.argtypes = [POINTER(c_uint64), _P]
    for name in ("gf_tile_grid", "gf_forward_bin", "gf_forward_emit", "gf_forward_render",
                 "gf_backward", "gf_backward_reduce", "gf_backward_finish", "gf_read_status",
                 "gf_selftest_softplus", "gf_batch_plan", "gf_batch_forward", "gf_batch_backward",
                 "gf_batch_set_grads", "gf_batch_read", "gf_backward_noalloc", "gf_forward",
                 "gf_backward_direct", "gf_fwd_bwd_fused", "gf_forward_kcap", "gf_backward_direct_kcap",
                 "gf_forward_bin_info", "gf_read_bin_info", "gf_backward_train"):
        getattr(L, name).restype = c_int
    _LIB = L
    return L


def check(rc: int, what: str) -> None:
    if rc != GF_OK:
        msg = lib().gf_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg} (code {rc})")


def ptr(t) -> int | None:
    """Device address of a tensor (None for an empty tensor)."""
    return t.data_ptr() if t is not None and t.numel() > 0 else None


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (as an integer)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)
