"""Drop-in for the reference's compiled extension module ``gaussian_peft_cuda_field_reference``.

Same three functions, argument order, return values and error messages as the pybind11
module (reference ``gaussian_peft/cuda_field/csrc/ext.cpp:9-110``); the work is done by
``libgaussfield.so`` through its C ABI (``include/gaussfield.h``).  Every call runs on
torch's *current* stream of the input device.

Host synchronisation: the forward reads the pair count P once (as the reference does at
``forward.cu:48-73``) to size ``gaussian_ids_sorted`` exactly; the same copy brings back the
widest Gaussian's tile count.  The backward reads one status word after its kernels to raise
the reference's saved-state errors (``field_impl.cu:86-108``); set ``VALIDATE_SAVED_STATE =
False`` to skip that read.

Backward kernels: given the forward workspace (the training Function passes it), int64 saved
state and no Gaussian over 320 tiles, the backward is the one-launch kernel plus a small kernel
that moves its gradients out (``gf_backward_train``); otherwise the reduction + finish.
"""

from __future__ import annotations

import contextlib
import ctypes

import torch
from torch import Tensor

from guass_amd import _native as N

VALIDATE_SAVED_STATE = True

# Host-side facts of a field, by (M, N, K, config): the tile count and the forward / backward
# workspace sizes (pure functions of the arguments; each costs a library call to compute).
_GEOMETRY: dict[tuple, tuple[int, int, int, int]] = {}
_CONFIGS: dict[tuple, N.GfFieldConfig] = {}
# The backward workspace, per (device, stream): zero at rest (every backward leaves its accumulators
# zero and its status word is cleared when read), so it is allocated and cleared once and reused.
# A call that fails drops it.
_BWD_WS: dict[tuple[int, int], Tensor] = {}


def _config(tile_out, tile_in, sigma_multiplier, normalize, clamp_quad) -> N.GfFieldConfig:
    key = (int(tile_out), int(tile_in), float(sigma_multiplier), bool(normalize),
           None if clamp_quad is None else float(clamp_quad))
    cfg = _CONFIGS.get(key)
    if cfg is None:
        cfg = _CONFIGS[key] = N.make_config(tile_out, tile_in, sigma_multiplier, normalize, clamp_quad)
    return cfg


def _geometry(M: int, Nf: int, K: int, cfg: N.GfFieldConfig) -> tuple[int, int, int, int]:
    """(R, C, forward workspace bytes, backward workspace bytes) of an M x N field of K Gaussians."""
    key = (M, Nf, K, cfg.tile_out, cfg.tile_in, cfg.sigma_multiplier, cfg.normalize, cfg.has_clamp_quad,
           cfg.clamp_quad)
    g = _GEOMETRY.get(key)
    if g is None:
        L = N.lib()
        R, C = ctypes.c_int64(), ctypes.c_int64()
        N.check(L.gf_tile_grid(M, Nf, ctypes.byref(cfg), ctypes.byref(R), ctypes.byref(C)), "gf_tile_grid")
        g = (R.value, C.value, int(L.gf_forward_workspace_bytes(M, Nf, K, ctypes.byref(cfg))),
             int(L.gf_backward_workspace_bytes(M, Nf, K, ctypes.byref(cfg))))
        if len(_GEOMETRY) > 4096:
            _GEOMETRY.clear()
        _GEOMETRY[key] = g
    return g


def _on_device(dev: torch.device):
    """torch.cuda.device(dev) unless dev is already the current device."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


# ------------------------------------------------------------------ checks (common.h:8-24)

def _check_cuda(t: Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _check_f32(t: Tensor, name: str) -> None:
    _check_cuda(t, name)
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32")


def _check_index(t: Tensor, name: str) -> None:
    _check_cuda(t, name)
    if t.dtype not in (torch.int32, torch.int64):
        raise RuntimeError(f"{name} must be int32 or int64")


def validate_forward_inputs(row_coords, col_coords, mu, chol_raw, amp) -> None:
    """field_impl.cu:52-71."""
    _check_f32(row_coords, "row_coords")
    _check_f32(col_coords, "col_coords")
    _check_f32(mu, "mu")
    _check_f32(chol_raw, "chol_raw")
    _check_f32(amp, "amp")
    if row_coords.dim() != 1:
        raise RuntimeError("row_coords must have shape [out_features]")
    if col_coords.dim() != 1:
        raise RuntimeError("col_coords must have shape [in_features]")
    if not (mu.dim() == 2 and mu.size(1) == 2):
        raise RuntimeError("mu must have shape [K, 2]")
    if not (chol_raw.dim() == 2 and chol_raw.size(1) == 3):
        raise RuntimeError("chol_raw must have shape [K, 3]")
    if not (amp.dim() == 2 and amp.size(1) == 1):
        raise RuntimeError("amp must have shape [K, 1]")
    if mu.size(0) != chol_raw.size(0):
        raise RuntimeError("mu and chol_raw must have the same K")
    if mu.size(0) != amp.size(0):
        raise RuntimeError("mu and amp must have the same K")


def _check_config(tile_out: int, tile_in: int, sigma_multiplier: float) -> None:
    """field_impl.cu:143-145."""
    if tile_out <= 0:
        raise RuntimeError("tile_out must be positive")
    if tile_in <= 0:
        raise RuntimeError("tile_in must be positive")
    if not sigma_multiplier > 0.0:
        raise RuntimeError("sigma_multiplier must be positive")


def _same_device(*ts: Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on the same device (got {dev} and {t.device})")
    return dev


# ------------------------------------------------------------------ forward

def gaussian_field_forward(row_coords: Tensor, col_coords: Tensor, mu: Tensor, chol_raw: Tensor,
                           amp: Tensor, tile_out: int, tile_in: int, sigma_multiplier: float,
                           normalize: bool, clamp_quad: float | None):
    """Returns (delta f32[M*N], tile_ptr i64[T+1], gaussian_ids_sorted i64[P])."""
    delta, tile_ptr, ids, _ = forward_with_workspace(row_coords, col_coords, mu, chol_raw, amp,
                                                     tile_out, tile_in, sigma_multiplier, normalize,
                                                     clamp_quad)
    return delta, tile_ptr, ids


def forward_with_workspace(row_coords: Tensor, col_coords: Tensor, mu: Tensor, chol_raw: Tensor,
                           amp: Tensor, tile_out: int, tile_in: int, sigma_multiplier: float,
                           normalize: bool, clamp_quad: float | None):
    """gaussian_field_forward plus its forward workspace, which holds the Gaussians' evaluation
    constants; passing it to gaussian_field_backward(forward_workspace=...) with the same
    parameters skips recomputing them."""
    validate_forward_inputs(row_coords, col_coords, mu, chol_raw, amp)
    _check_config(tile_out, tile_in, sigma_multiplier)
    dev = _same_device(row_coords, col_coords, mu, chol_raw, amp)
    M, Nf, K = row_coords.numel(), col_coords.numel(), mu.size(0)
    if M == 0 or Nf == 0:
        raise RuntimeError("out_features and in_features must be positive")
    L = N.lib()
    cfg = _config(tile_out, tile_in, sigma_multiplier, normalize, clamp_quad)
    R, C, ws_bytes, _ = _geometry(M, Nf, K, cfg)
    T = R * C
    pcfg = ctypes.byref(cfg)
    with _on_device(dev):
        stream = N.stream_handle(dev)
        # the device pair count lives in the 8 bytes after the workspace proper
        ws = torch.empty(ws_bytes + 256, dtype=torch.uint8, device=dev)
        ws_ptr = ws.data_ptr()
        tile_ptr = torch.empty(T + 1, dtype=torch.int64, device=dev)
        info = N.GfBinInfo()
        N.check(L.gf_forward_bin_info(pcfg, M, Nf, K, N.ptr(mu), N.ptr(chol_raw), N.ptr(amp),
                                      tile_ptr.data_ptr(), ws_ptr + ws_bytes, ctypes.byref(info),
                                      ws_ptr, ws_bytes, stream), "gaussian_field_forward (binning)")
        P = ctypes.c_int64(info.num_pairs)
        # the widest tile rectangle travels with the workspace: it picks the training backward's
        # kernels (gf_backward_train)
        ws.gf_max_span = int(info.max_span)
        ids = torch.empty(P.value, dtype=torch.int64, device=dev)
        delta = torch.empty(M * Nf, dtype=torch.float32, device=dev)
        N.check(L.gf_forward_emit(pcfg, M, Nf, K, N.ptr(mu), N.ptr(amp),
                                  tile_ptr.data_ptr(), N.ptr(ids), P.value, ws_ptr, ws_bytes,
                                  stream), "gaussian_field_forward (emit)")
        N.check(L.gf_forward_render(pcfg, M, Nf, K, row_coords.data_ptr(),
                                    col_coords.data_ptr(), tile_ptr.data_ptr(), N.ptr(ids), P.value,
                                    delta.data_ptr(), ws_ptr, ws_bytes, stream),
                "gaussian_field_forward (render)")
    return delta, tile_ptr, ids, ws


# ------------------------------------------------------------------ backward

_SAVED_STATE_MESSAGES = (  # order of the reference checks, field_impl.cu:92-106
    (N.GF_STATUS_TILE_PTR_LAST, "saved.tile_ptr[-1] must equal saved.gaussian_ids_sorted.numel()"),
    (N.GF_STATUS_TILE_PTR_ORDER, "saved.tile_ptr must be monotonic non-decreasing"),
    (N.GF_STATUS_IDS_NEGATIVE, "saved.gaussian_ids_sorted must be non-negative"),
    (N.GF_STATUS_IDS_RANGE, "saved.gaussian_ids_sorted contains out-of-range gaussian ids"),
)


def _backward(grad_delta, row_coords, col_coords, mu, chol_raw, amp, tile_ptr, gaussian_ids_sorted,
              tile_out, tile_in, sigma_multiplier, normalize, clamp_quad, forward_workspace):
    # validate_backward_inputs (field_impl.cu:73-84)
    _check_f32(grad_delta, "grad_delta")
    _check_f32(row_coords, "saved.row_coords")
    _check_f32(col_coords, "saved.col_coords")
    _check_f32(mu, "saved.mu")
    _check_f32(chol_raw, "saved.chol_raw")
    _check_f32(amp, "saved.amp")
    _check_index(tile_ptr, "saved.tile_ptr")
    _check_index(gaussian_ids_sorted, "saved.gaussian_ids_sorted")
    # validate_saved_state_contract, host part (field_impl.cu:87-91)
    if tile_ptr.dim() != 1:
        raise RuntimeError("saved.tile_ptr must have shape [num_tiles + 1]")
    if gaussian_ids_sorted.dim() != 1:
        raise RuntimeError("saved.gaussian_ids_sorted must have shape [num_pairs]")
    if tile_ptr.numel() < 1:
        raise RuntimeError("saved.tile_ptr must contain at least one element")
    _check_config(tile_out, tile_in, sigma_multiplier)
    M, Nf = row_coords.numel(), col_coords.numel()
    if grad_delta.numel() != M * Nf:
        raise RuntimeError("grad_delta must match flattened delta shape")
    if not (mu.dim() == 2 and mu.size(1) == 2 and chol_raw.dim() == 2 and chol_raw.size(1) == 3
            and amp.numel() == mu.size(0) and chol_raw.size(0) == mu.size(0)):
        raise RuntimeError("saved.mu / saved.chol_raw / saved.amp shapes disagree ([K,2], [K,3], [K,1])")
    dev = _same_device(grad_delta, row_coords, col_coords, mu, chol_raw, amp, tile_ptr,
                       gaussian_ids_sorted)
    K = mu.size(0)
    L = N.lib()
    cfg = _config(tile_out, tile_in, sigma_multiplier, normalize, clamp_quad)
    R, C, fwd_bytes, ws_bytes = _geometry(M, Nf, K, cfg)
    if tile_ptr.numel() != R * C + 1:
        raise RuntimeError(
            f"saved.tile_ptr has {tile_ptr.numel()} entries, expected num_tiles + 1 = "
            f"{R * C + 1} for a {M}x{Nf} field with {tile_out}x{tile_in} tiles")
    with _on_device(dev):
        stream = N.stream_handle(dev)
        key = (dev.index, stream)
        ws = _BWD_WS.pop(key, None) if VALIDATE_SAVED_STATE else None
        if ws is None or ws.numel() < ws_bytes:
            # zero-filled once; without the status read-back (which clears the status word) a
            # workspace is not reused
            ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
        fwd_ptr, max_span = None, -1
        if forward_workspace is not None:
            if (forward_workspace.device != dev or forward_workspace.dtype != torch.uint8
                    or forward_workspace.numel() < fwd_bytes):
                raise RuntimeError("forward_workspace does not belong to this field's forward")
            fwd_ptr = forward_workspace.data_ptr()
            max_span = int(getattr(forward_workspace, "gf_max_span", -1))
        d_mu = torch.empty(K, 2, dtype=torch.float32, device=dev)
        d_chol_raw = torch.empty(K, 3, dtype=torch.float32, device=dev)
        d_amp = torch.empty(K, 1, dtype=torch.float32, device=dev)
        # the one-launch kernel where the forward's binning allows it, else reduction + finish
        N.check(L.gf_backward_train(ctypes.byref(cfg), M, Nf, K, grad_delta.data_ptr(), row_coords.data_ptr(),
                                    col_coords.data_ptr(), N.ptr(mu), N.ptr(chol_raw), N.ptr(amp),
                                    tile_ptr.data_ptr(), int(tile_ptr.dtype == torch.int64),
                                    N.ptr(gaussian_ids_sorted), int(gaussian_ids_sorted.dtype == torch.int64),
                                    gaussian_ids_sorted.numel(), max_span, N.ptr(d_mu), N.ptr(d_chol_raw),
                                    N.ptr(d_amp), fwd_ptr, ws.data_ptr(), ws_bytes, stream),
                "gaussian_field_backward")
        if VALIDATE_SAVED_STATE:
            status = ctypes.c_uint32(0)
            # reads and clears the status word: the workspace is then zero again and kept
            N.check(L.gf_read_status(ws.data_ptr(), 1, ctypes.byref(status), stream), "gf_read_status")
            _BWD_WS[key] = ws
            for bit, msg in _SAVED_STATE_MESSAGES:
                if status.value & bit:
                    raise RuntimeError(msg)
    return [d_mu, d_chol_raw, d_amp]


def gaussian_field_backward(grad_delta: Tensor, row_coords: Tensor, col_coords: Tensor, mu: Tensor,
                            chol_raw: Tensor, amp: Tensor, tile_ptr: Tensor,
                            gaussian_ids_sorted: Tensor, tile_out: int, tile_in: int,
                            sigma_multiplier: float, normalize: bool, clamp_quad: float | None,
                            *, forward_workspace: Tensor | None = None):
    """Returns [d_mu f32[K,2], d_chol_raw f32[K,3], d_amp f32[K,1]].

    ``forward_workspace`` (keyword, optional): the workspace from ``forward_with_workspace`` over
    the same parameters, whose Gaussian constants are then reused."""
    return _backward(grad_delta, row_coords, col_coords, mu, chol_raw, amp, tile_ptr,
                     gaussian_ids_sorted, tile_out, tile_in, sigma_multiplier, normalize, clamp_quad,
                     forward_workspace)


def gaussian_field_backward_reference(grad_delta: Tensor, row_coords: Tensor, col_coords: Tensor,
                                      mu: Tensor, chol_raw: Tensor, amp: Tensor, tile_ptr: Tensor,
                                      gaussian_ids_sorted: Tensor, tile_out: int, tile_in: int,
                                      sigma_multiplier: float, normalize: bool,
                                      clamp_quad: float | None):
    """Validation entry (reference ext.cpp:73-110).  The reference's autograd replay cannot run
    (its delta has no grad_fn, backward.cu:500-539); this returns the same gradients as
    ``gaussian_field_backward``, which tests pin against the CPU autograd oracle."""
    return _backward(grad_delta, row_coords, col_coords, mu, chol_raw, amp, tile_ptr,
                     gaussian_ids_sorted, tile_out, tile_in, sigma_multiplier, normalize, clamp_quad,
                     None)
