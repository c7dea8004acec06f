"""gf_backward_noalloc: the backward with its workspace in the library's static device scratch.

Called through the C ABI and checked against the existing entry point gf_backward (same
kernels, a caller-allocated workspace) and against the CPU oracle, on consecutive calls of
shrinking size: a field with eight accumulator stripes, then cfg2, then cfg1.  Each call clears
only what it uses.  A call whose saved ids hold an id >= K leaves a status bit in the shared
scratch; the next clean call must report status 0 (its fill kernel cleared the word).  A HIP
graph captured over the entry point (after an eager call has looked up the scratch address)
replays to gf_backward's gradients.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from guass_amd import _native as N
from guass_amd import workloads as wl
from guass_amd.cuda_field import ext
from oracle import field_oracle as fo
from tests.parity import grad_close

GF_E_WORKSPACE = 2
SCRATCH_BYTES = 4 << 20


def _cfg():
    return N.make_config(16, 16, 3.0, False, 80.0)


def test_noalloc_rejects_fields_beyond_the_scratch():
    """A workspace past 4 MiB is refused with GF_E_WORKSPACE before any device work (safe
    without a GPU); gf_backward_workspace_bytes tells where the limit falls."""
    L = N.lib()
    cfg = ctypes.byref(_cfg())
    assert L.gf_backward_workspace_bytes(320, 768, 131064, cfg) == SCRATCH_BYTES
    assert L.gf_backward_workspace_bytes(320, 768, 131065, cfg) > SCRATCH_BYTES
    d = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    rc = L.gf_backward_noalloc(cfg, 320, 768, 131065, d, d, d, d, d, d, d, 1, d, 1, 1, d, d, d, None, None)
    assert rc == GF_E_WORKSPACE
    msg = L.gf_last_error().decode()
    assert "static scratch" in msg and "131064" in msg


def _noalloc(q, tp, ids, device):
    K = q.k
    out = [torch.full((K, n), float("nan"), dtype=torch.float32, device=device) for n in (2, 3, 1)]
    status = torch.full((1,), -1, dtype=torch.int32, device=device)
    N.check(N.lib().gf_backward_noalloc(
        ctypes.byref(_cfg()), q.out_features, q.in_features, K, q.grad.data_ptr(), q.row_coords.data_ptr(),
        q.col_coords.data_ptr(), q.mu.data_ptr(), q.chol_raw.data_ptr(), q.amp.data_ptr(), tp.data_ptr(),
        int(tp.dtype == torch.int64), ids.data_ptr(), int(ids.dtype == torch.int64), ids.numel(),
        out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), status.data_ptr(),
        N.stream_handle(device)), "gf_backward_noalloc")
    return out, status


@pytest.mark.gpu
def test_noalloc_backward_matches_gf_backward(device):
    probs = [wl.make_problem("stripes8_1280x1792_k512", 1280, 1792, 512, math.log(8.0), 0.6, 3),
             wl.cfg2(0), wl.cfg1(0)]
    for i, p in enumerate(probs):
        print(f"[gpu-test] gf_backward_noalloc call {i}: {p.name} M={p.out_features} N={p.in_features} K={p.k}",
              flush=True)
        q = p.to(device)
        _, tp, ids = ext.gaussian_field_forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, 16, 16, 3.0,
                                                False, 80.0)
        if i == 2:  # int32 saved state on the last call
            tp, ids = tp.to(torch.int32), ids.to(torch.int32)
        want = ext.gaussian_field_backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, tp, ids,
                                           16, 16, 3.0, False, 80.0)
        got, status = _noalloc(q, tp, ids, device)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        ref = fo.gaussian_field_fwd_bwd_batched(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad,
                                                16, 16, 3.0, False, 80.0)
        for name, a, b, r in zip(("d_mu", "d_chol_raw", "d_amp"), got, want, ref[3:]):
            grad_close(a, b, f"call {i} {name} vs gf_backward", rtol=1e-5)
            grad_close(a, r, f"call {i} {name} vs oracle")


@pytest.mark.gpu
def test_noalloc_status_cleared_between_calls(device):
    """A saved id >= K sets GF_STATUS_IDS_RANGE (the pair is skipped, no fault); the next clean
    call on the same scratch reports 0 and the oracle's gradients."""
    p = wl.cfg1(0)
    q = p.to(device)
    _, tp, ids = ext.gaussian_field_forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, 16, 16, 3.0,
                                            False, 80.0)
    bad = ids.clone()
    bad[-1] = p.k + 5
    print(f"[gpu-test] gf_backward_noalloc with an id >= K: {p.name}", flush=True)
    _, status = _noalloc(q, tp, bad, device)
    torch.cuda.synchronize()
    assert int(status.item()) & N.GF_STATUS_IDS_RANGE
    print(f"[gpu-test] gf_backward_noalloc clean call after it: {p.name}", flush=True)
    got, status = _noalloc(q, tp, ids, device)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    ref = fo.gaussian_field_fwd_bwd_batched(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad,
                                            16, 16, 3.0, False, 80.0)
    for name, a, r in zip(("d_mu", "d_chol_raw", "d_amp"), got, ref[3:]):
        grad_close(a, r, f"clean call {name} vs oracle")


@pytest.mark.gpu
def test_noalloc_backward_in_a_hip_graph(device):
    """gf_backward_noalloc captured in a HIP graph (its kernels only: the scratch address was
    looked up by an eager call) and replayed three times, with eager work, NaN-filled outputs and
    synchronisations between the replays: every replay equals gf_backward's gradients."""
    p = wl.cfg2(1)
    q = p.to(device)
    _, tp, ids = ext.gaussian_field_forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, 16, 16, 3.0,
                                            False, 80.0)
    want = ext.gaussian_field_backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, tp, ids,
                                       16, 16, 3.0, False, 80.0)
    print(f"[gpu-test] gf_backward_noalloc eager call before capture: {p.name}", flush=True)
    _noalloc(q, tp, ids, device)
    K = p.k
    out = [torch.empty((K, n), dtype=torch.float32, device=device) for n in (2, 3, 1)]
    status = torch.empty((1,), dtype=torch.int32, device=device)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("[gpu-test] capturing gf_backward_noalloc", flush=True)
    with torch.cuda.graph(graph):
        N.check(N.lib().gf_backward_noalloc(
            ctypes.byref(_cfg()), q.out_features, q.in_features, K, q.grad.data_ptr(), q.row_coords.data_ptr(),
            q.col_coords.data_ptr(), q.mu.data_ptr(), q.chol_raw.data_ptr(), q.amp.data_ptr(), tp.data_ptr(), 1,
            ids.data_ptr(), 1, ids.numel(), out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(),
            status.data_ptr(), N.stream_handle(device)), "gf_backward_noalloc (captured)")
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"[gpu-test]   replay {rep}", flush=True)
        junk = torch.randn(1 << 16, device=device)
        float(junk.sum())  # eager work and a synchronisation between the replays
        for t in out:
            t.fill_(float("nan"))
        status.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert int(status.item()) == 0, f"replay {rep}: status"
        for name, a, b in zip(("d_mu", "d_chol_raw", "d_amp"), out, want):
            grad_close(a, b, f"replay {rep} {name} vs gf_backward", rtol=1e-5)
