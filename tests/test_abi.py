"""The C ABI and the drop-in shim without a GPU.

* libgaussfield.so loads and exports every function include/gaussfield.h declares (and the
  ctypes binding declares the same set);
* host-side argument validation returns the documented GF_E_* codes and messages before any
  device work, so these calls are safe on a machine without a GPU;
* the drop-in ``ext`` functions raise the reference's error messages for non-CUDA inputs and
  bad configurations (common.h:8-24, field_impl.cu:52-71,143-145);
* the runtime exports the names GaussianLinear and the patchers import (cuda_field/__init__.py).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from guass_amd import _native as N

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "gaussfield.h"

GF_E_INVALID_ARGUMENT = 1
GF_E_WORKSPACE = 2


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^[A-Za-z_][\w \t\*]*?\b(gf_\w+)\s*\(", text, flags=re.M))


def test_header_error_codes():
    text = HEADER.read_text()
    assert re.search(r"#define\s+GF_E_INVALID_ARGUMENT\s+1\b", text)
    assert re.search(r"#define\s+GF_E_WORKSPACE\s+2\b", text)
    for name in ("CAPACITY", "COUNT_MISMATCH", "TILE_PTR_LAST", "TILE_PTR_ORDER", "IDS_NEGATIVE",
                 "IDS_RANGE"):
        m = re.search(rf"#define\s+GF_STATUS_{name}\s+(0x[0-9a-fA-F]+)u", text)
        assert m and int(m.group(1), 16) == getattr(N, f"GF_STATUS_{name}"), name


def test_library_exports_every_declared_symbol():
    declared = declared_functions()
    assert len(declared) >= 13
    assert declared == set(N.EXPORTED)
    lib = N.lib()
    for name in sorted(declared):
        assert hasattr(lib, name), f"{name} declared in include/gaussfield.h but not exported"
    assert lib.gf_version().decode().startswith("gaussfield-mi355x")


def _cfg(**kw):
    base = dict(tile_out=16, tile_in=16, sigma_multiplier=3.0, normalize=False, clamp_quad=80.0)
    base.update(kw)
    return N.make_config(**base)


def test_tile_grid_and_workspace_sizes():
    lib = N.lib()
    R, C = ctypes.c_int64(), ctypes.c_int64()
    assert lib.gf_tile_grid(1280, 5120, ctypes.byref(_cfg()), ctypes.byref(R), ctypes.byref(C)) == 0
    assert (R.value, C.value) == (80, 320)
    assert lib.gf_tile_grid(45, 70, ctypes.byref(_cfg(tile_out=8, tile_in=24)), ctypes.byref(R),
                            ctypes.byref(C)) == 0
    assert (R.value, C.value) == (6, 3)
    fwd = lib.gf_forward_workspace_bytes(1280, 1280, 1024, ctypes.byref(_cfg()))
    bwd = lib.gf_backward_workspace_bytes(1280, 1280, 1024, ctypes.byref(_cfg()))
    # header + 32 B constants + 16 B rectangle per Gaussian + 4 B fill counter per tile; 32 B
    # per Gaussian of accumulators
    assert fwd >= 256 + 48 * 1024 + 4 * 6400 and fwd % 256 == 0
    assert bwd >= 256 + 32 * 1024 and bwd % 256 == 0
    assert lib.gf_forward_workspace_bytes(10, 10, 4, ctypes.byref(_cfg(tile_out=0))) == 0


@pytest.mark.parametrize("shape,kc", [((1280, 1280), 9000), ((320, 768), 8500), ((96, 80), 300),
                                      ((1280, 1280), 5000)])
def test_forward_workspace_bytes_max_is_worst_case(shape, kc):
    """gf_forward_workspace_bytes_max(kc) = the largest gf_forward_workspace_bytes over every
    K in [0, kc], by brute force.  Past K = 8192 the masks drop out and the need falls, so for
    kc > 8192 the worst case is an interior K, not kc."""
    lib = N.lib()
    cfg = ctypes.byref(_cfg())
    M, Nf = shape
    need = [lib.gf_forward_workspace_bytes(M, Nf, k, cfg) for k in range(kc + 1)]
    assert lib.gf_forward_workspace_bytes_max(M, Nf, kc, cfg) == max(need)
    if kc > 8192:
        assert max(need) > need[kc]
    assert lib.gf_forward_workspace_bytes_max(M, Nf, -1, cfg) == 0


@pytest.mark.parametrize("kw,msg", [({"tile_out": 0}, "tile_out must be positive"),
                                    ({"tile_in": -2}, "tile_in must be positive"),
                                    ({"sigma_multiplier": 0.0}, "sigma_multiplier must be positive")])
def test_invalid_config_is_rejected_before_device_work(kw, msg):
    lib = N.lib()
    R, C = ctypes.c_int64(), ctypes.c_int64()
    rc = lib.gf_tile_grid(64, 64, ctypes.byref(_cfg(**kw)), ctypes.byref(R), ctypes.byref(C))
    assert rc == GF_E_INVALID_ARGUMENT
    assert msg in lib.gf_last_error().decode()
    # the same check guards every entry point that takes a config
    rc = lib.gf_forward_bin(ctypes.byref(_cfg(**kw)), 64, 64, 4, None, None, None, None, None,
                            None, None, 0, None)
    assert rc == GF_E_INVALID_ARGUMENT and msg in lib.gf_last_error().decode()


def test_workspace_and_pointer_checks():
    lib = N.lib()
    cfg = _cfg()
    need = lib.gf_forward_workspace_bytes(64, 64, 4, ctypes.byref(cfg))
    rc = lib.gf_forward_bin(ctypes.byref(cfg), 64, 64, 4, None, None, None, None, None, None, None,
                            need - 1, None)
    assert rc == GF_E_WORKSPACE and "workspace" in lib.gf_last_error().decode()
    rc = lib.gf_tile_grid(0, 64, ctypes.byref(cfg), None, None)
    assert rc == GF_E_INVALID_ARGUMENT
    rc = lib.gf_tile_grid(64, 64, None, None, None)
    assert rc == GF_E_INVALID_ARGUMENT
    rc = lib.gf_read_status(None, 0, None, None)
    assert rc == GF_E_INVALID_ARGUMENT


def test_backward_direct_host_logic():
    """gf_backward_direct's host side: the launch count it will make (1 on the mask path with
    sparse 16x16 / 32x32 tiles, heavy tiles included, below 8192 tiles or with the widest
    rectangle known, and no known rectangle of 320 tiles or more; 2 elsewhere), where its
    gradient slots lie in the forward workspace, and the workspace check before any device
    work."""
    lib = N.lib()
    cfg = ctypes.byref(_cfg())

    def launches(M, Nf, K, P, c=cfg, span=-1):
        return lib.gf_backward_direct_launches(c, M, Nf, K, P, span)

    # the widest rectangle: one Gaussian's atomics serialise on its slot
    assert launches(1280, 1280, 1024, 23618, span=15) == 1
    assert launches(1280, 1280, 1024, 23618, span=319) == 1
    assert launches(1280, 1280, 1024, 23618, span=320) == 2
    assert launches(1280, 1280, 1024, 30003, span=6400) == 2
    assert launches(1280, 1280, 1024, 30003, span=-1) == 1  # not known: the shape decides

    assert launches(1280, 1280, 1024, 23618) == 1          # cfg3
    assert launches(1280, 1280, 1024, 16 * 6400) == 2      # dense tiles: the transposing reduction
    assert launches(1280, 1280, 1024, 12 * 6400, span=9) == 1  # 8..16 a tile: still one launch (row sums)
    assert launches(1280, 1792, 512, 20000) == 2           # 8960 tiles, widest rectangle not known
    assert launches(1280, 1792, 512, 20000, span=100) == 1  # ... known to be narrow
    assert launches(1280, 1792, 512, 20000, span=400) == 2
    assert launches(1280, 1280, 2048, 40000) == 1          # heavy-tile workgroups add into the slots too
    assert launches(1280, 5120, 4096, 52094, span=90) == 1  # cfg5c: heavy tiles, 25600 tiles
    assert launches(320, 320, 9000, 20000) == 2            # past the masks: the emission path
    assert launches(320, 768, 256, 2000) == 1              # cfg2, binned in the render
    assert launches(1280, 1280, 1024, 23618, ctypes.byref(_cfg(tile_out=32, tile_in=32))) == 1
    assert launches(200, 200, 100, 500, ctypes.byref(_cfg(tile_out=8, tile_in=8))) == 2
    assert launches(64, 64, 0, 0) == 2
    assert launches(64, 64, 4, 10, ctypes.byref(_cfg(tile_out=0))) == -GF_E_INVALID_ARGUMENT
    for M, Nf, K in ((1280, 1280, 1024), (320, 768, 256), (45, 70, 9000)):
        off = lib.gf_forward_grads_offset(M, Nf, K, cfg)
        total = lib.gf_forward_workspace_bytes(M, Nf, K, cfg)
        assert off % 256 == 0 and 256 <= off and off + 32 * K <= total
    need = lib.gf_forward_workspace_bytes(64, 64, 4, cfg)
    rc = lib.gf_backward_direct(cfg, 64, 64, 4, None, None, None, None, None, None, None, None, 10, -1, None,
                                need, None, 0, None)
    assert rc == GF_E_WORKSPACE and "forward workspace" in lib.gf_last_error().decode()
    rc = lib.gf_backward_direct(cfg, 64, 64, 4, None, None, None, None, None, None, None, None, 10, -1, 256,
                                need - 1, None, 0, None)
    assert rc == GF_E_WORKSPACE


def test_bin_info_and_train_backward_host_checks():
    """gf_forward_bin_info / gf_read_bin_info refuse NULL outputs, and gf_backward_train checks
    its field and buffers before any device work on either of its paths (safe without a GPU)."""
    lib = N.lib()
    cfg = _cfg()
    need = lib.gf_forward_workspace_bytes(64, 64, 4, ctypes.byref(cfg))
    rc = lib.gf_forward_bin_info(ctypes.byref(cfg), 64, 64, 4, None, None, None, None, None, None, None, need, None)
    assert rc == GF_E_INVALID_ARGUMENT and "info" in lib.gf_last_error().decode()
    info = N.GfBinInfo()
    rc = lib.gf_forward_bin_info(ctypes.byref(cfg), 64, 64, 4, None, None, None, None, None, ctypes.byref(info),
                                 None, need - 1, None)
    assert rc == GF_E_WORKSPACE
    assert lib.gf_read_bin_info(None, ctypes.byref(info), None) == GF_E_INVALID_ARGUMENT
    assert lib.gf_read_bin_info(ctypes.c_void_p(256), None, None) == GF_E_INVALID_ARGUMENT
    rc = lib.gf_backward_train(ctypes.byref(_cfg(tile_out=0)), 64, 64, 4, None, None, None, None, None, None,
                               None, 1, None, 1, 10, 15, None, None, None, None, None, 0, None)
    assert rc == GF_E_INVALID_ARGUMENT and "tile_out must be positive" in lib.gf_last_error().decode()
    # the one-launch path (mask path, sparse, span known and small) checks its backward workspace
    d = ctypes.c_void_p(256)  # never dereferenced: the workspace check comes first
    rc = lib.gf_backward_train(ctypes.byref(cfg), 64, 64, 4, d, d, d, d, d, d, d, 1, d, 1, 10, 15, d, d, d, d,
                               None, 0, None)
    assert rc == GF_E_WORKSPACE and "backward workspace" in lib.gf_last_error().decode()
    # the reduction path (span not known) likewise
    rc = lib.gf_backward_train(ctypes.byref(cfg), 64, 64, 4, d, d, d, d, d, d, d, 1, d, 1, 10, -1, d, d, d, d,
                               None, 0, None)
    assert rc == GF_E_WORKSPACE


def test_shim_rejects_cpu_tensors_with_reference_messages():
    from guass_amd.cuda_field import ext

    M, Nn, K = 32, 48, 3
    rc, cc = torch.linspace(-1, 1, M), torch.linspace(-1, 1, Nn)
    mu, raw, amp = torch.zeros(K, 2), torch.zeros(K, 3), torch.zeros(K, 1)
    with pytest.raises(RuntimeError, match="row_coords must be a CUDA tensor"):
        ext.gaussian_field_forward(rc, cc, mu, raw, amp, 16, 16, 3.0, False, 80.0)
    grad = torch.zeros(M * Nn)
    tp, ids = torch.zeros(7, dtype=torch.int64), torch.zeros(0, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="grad_delta must be a CUDA tensor"):
        ext.gaussian_field_backward(grad, rc, cc, mu, raw, amp, tp, ids, 16, 16, 3.0, False, 80.0)
    with pytest.raises(RuntimeError, match="grad_delta must be a CUDA tensor"):
        ext.gaussian_field_backward_reference(grad, rc, cc, mu, raw, amp, tp, ids, 16, 16, 3.0,
                                              False, 80.0)


def test_runtime_surface():
    from guass_amd import cuda_field
    from guass_amd.cuda_field import contracts, runtime

    for name in ("gaussian_field_train", "gaussian_field_reference", "gaussian_field_forward_reference",
                 "gaussian_field_cuda_field_stage2_validation", "load_extension"):
        assert callable(getattr(cuda_field, name)), name
    assert issubclass(runtime.GaussianFieldCudaTrainFunction, torch.autograd.Function)
    assert issubclass(runtime.GaussianFieldCudaReferenceFunction, torch.autograd.Function)
    th = contracts.CudaFieldStage0Thresholds()
    assert th.default_sigma_multiplier == 3.0 and th.partial_grad_bytes_limit == 256 * 1024 * 1024
    ext = cuda_field.load_extension()
    for name in ("gaussian_field_forward", "gaussian_field_backward", "gaussian_field_backward_reference"):
        assert callable(getattr(ext, name)), name


def test_saved_tensor_spec_field_order():
    """CudaFieldSavedTensorSpec declares its fields in the reference's order (contracts.py:34-46);
    SAVED_TENSOR_ORDER is the save_for_backward order (runtime.py:148-156)."""
    import dataclasses

    from guass_amd.cuda_field import contracts

    names = [f.name for f in dataclasses.fields(contracts.CudaFieldSavedTensorSpec)]
    assert names == ["mu", "chol_raw", "amp", "row_coords", "col_coords", "tile_ptr", "gaussian_ids_sorted"]
    assert all(getattr(contracts.SAVED_TENSOR_SPEC, n) == n for n in names)
    assert contracts.SAVED_TENSOR_ORDER == ("row_coords", "col_coords", "mu", "chol_raw", "amp", "tile_ptr",
                                            "gaussian_ids_sorted")


def test_train_function_backward_notice_once(monkeypatch):
    """The training Function emits its backward notice once per process and keeps
    _backward_warning_emitted (reference runtime.py:119,165-174).  Runs on the CPU with a
    stand-in extension that records the calls (no kernels)."""
    import warnings

    from guass_amd.cuda_field import runtime

    class _Ext:
        calls = []

        def forward_with_workspace(self, row_coords, col_coords, mu, chol_raw, amp, *cfg):
            self.calls.append("forward")
            n = row_coords.numel() * col_coords.numel()
            return (torch.zeros(n), torch.zeros(2, dtype=torch.int64), torch.zeros(0, dtype=torch.int64),
                    torch.zeros(1, dtype=torch.uint8))

        def gaussian_field_backward(self, grad, row_coords, col_coords, mu, chol_raw, amp, tile_ptr, ids, *cfg,
                                    forward_workspace=None):
            self.calls.append("backward")
            return [torch.ones_like(mu), torch.ones_like(chol_raw), torch.ones_like(amp)]

    stub = _Ext()
    monkeypatch.setattr(runtime, "load_extension", lambda verbose=False: stub)
    monkeypatch.setattr(runtime.GaussianFieldCudaTrainFunction, "_backward_warning_emitted", False)
    mu = torch.zeros(3, 2, requires_grad=True)
    raw = torch.zeros(3, 3, requires_grad=True)
    amp = torch.zeros(3, 1, requires_grad=True)
    seen = []
    for _ in range(2):
        delta = runtime.gaussian_field_train(row_coords=torch.zeros(4), col_coords=torch.zeros(5), mu=mu,
                                             chol_raw=raw, amp=amp, tile_out=16, tile_in=16, sigma_multiplier=3.0)
        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always")
            delta.sum().backward()
        seen.append(sum("gaussian_field_train uses the active custom CUDA backward path" in str(w.message)
                        for w in caught))
    assert seen == [1, 0]
    assert runtime.GaussianFieldCudaTrainFunction._backward_warning_emitted
    assert stub.calls == ["forward", "backward", "forward", "backward"]
    assert torch.equal(mu.grad, torch.full((3, 2), 2.0))


# names exported by gaussian_peft/cuda_field/__init__.py:20-35
REFERENCE_CUDA_FIELD_ALL = (
    "CUDA_FIELD_EXTENSION_NAME", "CUDA_FIELD_REFERENCE_EXTENSION_NAME", "CUDA_FIELD_SOURCES",
    "GaussianFieldCudaFunctionStage0", "NON_DIFFERENTIABLE_ARGS", "SAVED_TENSOR_SPEC",
    "STAGE0_THRESHOLDS", "TENSOR_CONTRACT", "build_instructions", "gaussian_field_forward_reference",
    "gaussian_field_reference", "gaussian_field_train", "get_source_paths", "load_extension",
)


def test_package_surface_covers_reference_names():
    from guass_amd import cuda_field

    missing = [n for n in REFERENCE_CUDA_FIELD_ALL if not hasattr(cuda_field, n)]
    assert not missing, missing
    assert set(REFERENCE_CUDA_FIELD_ALL) <= set(cuda_field.__all__)
    with pytest.raises(NotImplementedError):
        cuda_field.GaussianFieldCudaFunctionStage0.forward(None, *([None] * 10))


def test_product_path_has_no_cpu_fallback(monkeypatch, tmp_path):
    """Without the built library the product path raises instead of computing anything."""
    monkeypatch.setattr(N, "_LIB", None)
    monkeypatch.setattr(N, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        N.lib()


def _batch_info(layers_mnk, *, tile=16, k_capacity=0):
    """gf_batch_plan's size query (host only: no device memory is touched) for layers of the
    given (out, in, k); the pointer fields hold placeholder addresses."""
    lib = N.lib()
    cfg = _cfg(tile_out=tile, tile_in=tile)
    fake = 0x10000
    table = (N.GfLayer * len(layers_mnk))()
    for i, (m, n, k) in enumerate(layers_mnk):
        fwd = lib.gf_forward_workspace_bytes(m, n, k, ctypes.byref(cfg))
        bwd = lib.gf_backward_workspace_bytes(m, n, k, ctypes.byref(cfg))
        table[i] = N.GfLayer(m, n, k, fake, fake, fake, fake, fake, fake, fake, fake, fake, 1, fake, fwd,
                             None, fake, fake, fake, fake, bwd, k_capacity)
    info = N.GfBatchInfo()
    rc = lib.gf_batch_plan(ctypes.byref(cfg), table, len(layers_mnk), None, 0, ctypes.byref(info), None)
    assert rc == 0, lib.gf_last_error().decode()
    return (info.tile_blocks, info.emit_blocks, info.finish_blocks, info.render_blocks, info.tile_render,
            info.plan_bytes)


@pytest.mark.parametrize("tile", [16, 32])
def test_batch_plan_grids_fixed_within_k_capacity(tile):
    """Densification changes K (reference controllers/clone.py:31-56, prune.py:34-45): with
    k_capacity the launch grids and the plan size do not depend on K up to the capacity, so a
    plan re-written in place keeps graph-captured launches valid; without it they follow K."""
    shapes = [(320, 320), (320, 768), (1280, 1280)]
    ref = _batch_info([(m, n, 1024) for m, n in shapes], tile=tile, k_capacity=1024)
    for ks in ([256, 257, 1000], [1, 1024, 513], [1024, 1024, 1024]):
        got = _batch_info([(m, n, k) for (m, n), k in zip(shapes, ks)], tile=tile, k_capacity=1024)
        assert got == ref, ks
    small = _batch_info([(m, n, 256) for m, n in shapes], tile=tile)
    assert small[2] < ref[2]  # finish blocks follow K without a capacity
    assert small[0] == ref[0]  # tile blocks depend on the tile grid only


def test_batch_plan_reserves_emission_blocks_for_capacity():
    """A layer whose capacity lies past the mask path (K > 8192) keeps emit blocks while its
    current K is on the mask path; their workgroups return at once (k_emit_batch)."""
    mask = _batch_info([(320, 320, 4096)])
    assert mask[1] == 0
    reserved = _batch_info([(320, 320, 4096)], k_capacity=16384)
    emitting = _batch_info([(320, 320, 16384)], k_capacity=16384)
    assert reserved[1] > 0 and reserved == emitting
    lib = N.lib()
    cfg = _cfg()
    table = (N.GfLayer * 1)()
    table[0] = N.GfLayer(64, 64, 4, *([0x10000] * 9), 1, 0x10000, 1 << 20, None, *([0x10000] * 4), 1 << 20, -1)
    info = N.GfBatchInfo()
    rc = lib.gf_batch_plan(ctypes.byref(cfg), table, 1, None, 0, ctypes.byref(info), None)
    assert rc == GF_E_INVALID_ARGUMENT and "k_capacity" in lib.gf_last_error().decode()


def test_fused_entry_refuses_other_fields_before_device_work():
    """gf_fwd_bwd_fused takes 16x16 tiles on the mask path, fewer than 8192 tiles, sparse fields
    without heavy tiles (gf_fwd_bwd_fused_supported); other fields are refused with
    GF_E_INVALID_ARGUMENT before any device work (safe without a GPU)."""
    L = N.lib()
    c16, c32 = N.make_config(16, 16, 3.0, False, 80.0), N.make_config(32, 32, 3.0, False, 80.0)
    ok = lambda cfg, m, n, k, cap, span=-1: L.gf_fwd_bwd_fused_supported(ctypes.byref(cfg), m, n, k, cap,  # noqa: E731
                                                                          span)
    assert ok(c16, 1280, 1280, 1024, 24000) == 1
    assert ok(c16, 1280, 1280, 1024, 24000, 100) == 1
    assert ok(c16, 1280, 1280, 1024, 24000, 320) == 0       # a known rectangle of 320 tiles or more
    assert ok(c16, 320, 320, 64, 500) == 1
    assert ok(c32, 1280, 1280, 1024, 24000) == 0          # 32x32 tiles
    assert ok(c16, 320, 320, 9000, 9000) == 0             # past the masks: emission path
    assert ok(c16, 1280, 1792, 512, 4000) == 0            # 8960 tiles
    assert ok(c16, 320, 320, 600, 16 * 400) == 0          # dense (>= 16 pairs a tile)
    assert ok(c16, 640, 640, 2048, 20000) == 0            # heavy-tile workgroups
    assert ok(c16, 320, 320, 0, 1) == 0                   # no Gaussian
    d = ctypes.c_void_p(16)  # never dereferenced: the field is refused first
    rc = L.gf_fwd_bwd_fused(ctypes.byref(c32), 1280, 1280, 1024, d, d, d, d, d, d, d, d, d, 24000, d, d, 1 << 30,
                            None)
    assert rc == GF_E_INVALID_ARGUMENT
    assert "gf_fwd_bwd_fused_supported" in L.gf_last_error().decode()
