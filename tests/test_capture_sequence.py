"""The library calls a GaussianFieldBatch training step makes, recorded on the CPU.

A step of ``render(check=False)``, every layer's forward and autograd's backward is what a caller
would capture in a HIP graph (reference step: gaussian_peft/trainers/base_trainer.py:71-90).  Here
``libgaussfield.so`` is replaced by a recording stand-in (no kernels run) and the step runs on CPU
tensors, so the test pins what the Python side asks of the library inside that region:

* only the three launch entries ``gf_batch_forward``, ``gf_batch_set_grads`` and
  ``gf_batch_backward`` are reached -- no ``gf_batch_plan`` (which uploads the layer table and
  synchronises), no ``gf_batch_read`` / ``gf_read_status`` (read-backs);
* every launch goes to the stream that is current, on the thread that makes it, at the time of
  the call (inside a capture that is the capture stream; autograd's backward thread sets it);
* nothing in the region reads a tensor back to the host (``.item()``, ``.tolist()``,
  ``float(t)``, ``.cpu()``, ``.numpy()``) or allocates a zero-filled buffer for a missing
  gradient (``torch.zeros``) when every layer's forward ran.
"""

from __future__ import annotations

import ctypes
import threading

import pytest
import torch

from guass_amd import _native as N
from guass_amd.layers import GaussianAdapterConfig, GaussianFieldBatch, GaussianLinear

LAUNCHES = {"gf_batch_forward", "gf_batch_set_grads", "gf_batch_backward"}


class RecordingLib:
    """Stand-in for the ctypes library: host-side answers of the right shape, a record of every
    call as (name, thread id, stream argument)."""

    def __init__(self):
        self.calls: list[tuple[str, int, int | None]] = []

    def _rec(self, name, stream=None):
        self.calls.append((name, threading.get_ident(), stream))

    def gf_last_error(self):
        return b"recording stand-in"

    def gf_tile_grid(self, m, n, cfg, r, c):
        self._rec("gf_tile_grid")
        r._obj.value, c._obj.value = (m + 15) // 16, (n + 15) // 16
        return 0

    def gf_forward_workspace_bytes(self, m, n, k, cfg):
        return 1024 + 64 * k

    def gf_forward_workspace_bytes_max(self, m, n, kc, cfg):
        return 1024 + 64 * kc

    def gf_backward_workspace_bytes(self, m, n, k, cfg):
        return 512 + 32 * k

    def gf_batch_plan(self, cfg, table, n, plan, plan_bytes, info, stream):
        self._rec("gf_batch_plan", stream)
        inf = info._obj
        inf.n_layers, inf.plan_bytes, inf.backward_buffers = n, 4096, 1
        inf.tile_blocks, inf.render_blocks, inf.finish_blocks = 8 * n, 4 * n, n
        inf.has_backward = 0
        return 0

    def gf_batch_forward(self, plan, info, phases, stream):
        self._rec("gf_batch_forward", stream)
        return 0

    def gf_batch_set_grads(self, plan, info, ptrs, stream):
        self._rec("gf_batch_set_grads", stream)
        info._obj.has_backward = info._obj.backward_buffers
        return 0

    def gf_batch_backward(self, plan, info, phases, stream):
        self._rec("gf_batch_backward", stream)
        return 0 if info._obj.has_backward else 1

    def gf_batch_read(self, plan, info, clear, status, pairs, norms, stream):
        self._rec("gf_batch_read", stream)
        for i in range(info._obj.n_layers):
            status[i], pairs[i] = 0, 40
            if norms is not None:
                norms[i] = 1.0
        return 0

    def gf_read_status(self, ws, clear, status, stream):
        self._rec("gf_read_status", stream)
        return 0


@pytest.fixture
def recording(monkeypatch):
    lib = RecordingLib()
    monkeypatch.setattr(N, "_LIB", lib)
    current: dict[int, int] = {}

    def stream_handle(device):
        # a distinct stream value per thread, so a launch made with another thread's stream shows
        return current.setdefault(threading.get_ident(), 0x1000 + len(current))

    monkeypatch.setattr(N, "stream_handle", stream_handle)
    return lib, current


class HostReads:
    """Counts host read-backs and zero-filled allocations while active."""

    NAMES = ("item", "tolist", "__float__", "__int__", "cpu", "numpy")

    def __init__(self, monkeypatch):
        self.seen: list[str] = []
        self.active = False
        for name in self.NAMES:
            orig = getattr(torch.Tensor, name)

            def wrap(self_t, *a, _orig=orig, _name=name, **k):
                if self.active:
                    self.seen.append(_name)
                return _orig(self_t, *a, **k)

            monkeypatch.setattr(torch.Tensor, name, wrap)
        orig_zeros = torch.zeros

        def zeros(*a, **k):
            if self.active:
                self.seen.append("torch.zeros")
            return orig_zeros(*a, **k)

        monkeypatch.setattr(torch, "zeros", zeros)


def _layers(shapes, delta_apply):
    torch.manual_seed(3)
    out = []
    for n_in, n_out, k in shapes:
        cfg = GaussianAdapterConfig(init_num_gaussians=k, tile_out=16, tile_in=16, adapter_scale=0.5,
                                    delta_apply=delta_apply)
        out.append(GaussianLinear(n_in, n_out, adapter_config=cfg))
    return out


@pytest.mark.parametrize("delta_apply", ["row_chunk", "merged"])
def test_unchecked_step_reaches_only_launch_entries(recording, monkeypatch, delta_apply):
    lib, current = recording
    shapes = [(96, 80, 48), (64, 64, 24), (120, 40, 36)]
    layers = _layers(shapes, delta_apply)
    xs = [torch.randn(6, n_in) for n_in, _, _ in shapes]
    gys = [torch.randn(6, n_out) for _, n_out, _ in shapes]
    fb = GaussianFieldBatch(layers)
    reads = HostReads(monkeypatch)

    def step(check):
        for ly in layers:
            for t in ly.get_gaussian_parameters().values():
                t.grad = None
        fb.render(check=check)
        torch.autograd.backward([ly(x) for ly, x in zip(layers, xs)], gys)

    step(True)  # plans and reads back (outside the region a caller would capture)
    eager = [name for name, _, _ in lib.calls]
    assert "gf_batch_plan" in eager and "gf_batch_read" in eager
    for _ in range(2):  # the region: twice, as a warm-up and a capture would run it
        lib.calls.clear()
        reads.active = True
        step(False)
        reads.active = False
        names = [name for name, _, _ in lib.calls]
        assert names == ["gf_batch_forward", "gf_batch_set_grads", "gf_batch_backward"], names
        assert reads.seen == [], reads.seen
        for name, tid, stream in lib.calls:
            assert stream == current[tid], f"{name} launched on another thread's stream"
        assert all(t.grad is not None for ly in layers for t in ly.get_gaussian_parameters().values())
    assert fb.replans == 0


def test_unchecked_step_with_an_idle_layer_allocates_its_zero_gradient_once(recording, monkeypatch):
    """A layer whose forward does not run gets a zero dL/d(delta-W): allocated at its first such
    backward and kept, so a later step reuses the buffer (no allocation inside a replayed step)."""
    lib, _ = recording
    shapes = [(96, 80, 48), (64, 64, 24)]
    layers = _layers(shapes, "row_chunk")
    x = torch.randn(6, 96)
    gy = torch.randn(6, 80)
    fb = GaussianFieldBatch(layers)
    reads = HostReads(monkeypatch)
    fb.render()
    layers[0](x).backward(gy)  # layer 1 idle: its zero gradient is allocated here
    layers[1]._batched_delta = None
    for _ in range(2):
        lib.calls.clear()
        reads.active = True
        fb.render(check=False)
        layers[0](x).backward(gy)
        reads.active = False
        layers[1]._batched_delta = None
        assert [n for n, _, _ in lib.calls] == ["gf_batch_forward", "gf_batch_set_grads", "gf_batch_backward"]
        assert reads.seen == [], reads.seen


def test_recording_lib_answers_ctypes_calls():
    """The stand-in accepts the ctypes argument forms the package passes (byref structures and
    arrays)."""
    lib = RecordingLib()
    r, c = ctypes.c_int64(), ctypes.c_int64()
    assert lib.gf_tile_grid(40, 33, None, ctypes.byref(r), ctypes.byref(c)) == 0
    assert (r.value, c.value) == (3, 3)
    info = N.GfBatchInfo()
    assert lib.gf_batch_plan(None, None, 2, None, 0, ctypes.byref(info), 7) == 0
    assert info.n_layers == 2 and info.plan_bytes == 4096
