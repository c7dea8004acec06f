"""Sync-free, allocation-free-per-call use of libgaussfield.so.

``FieldPlan`` owns every device buffer of one layer's forward and backward (workspaces,
tile_ptr, a gaussian-id buffer of fixed capacity, delta-W and the gradients), so a training
step issues kernels only -- no host synchronisation and no allocation -- and can be captured
in a HIP graph.  The pair count is not read back: if it ever exceeds the id capacity the
kernels set ``GF_STATUS_CAPACITY`` (check with ``status()``), and the caller re-plans with a
larger capacity.
"""

from __future__ import annotations

import ctypes

import torch

from guass_amd import _native as N


class FieldPlan:
    """Device buffers of one field's forward and backward, sized for ``k_capacity`` Gaussians
    (default ``k``): :meth:`resize` moves to another K (densification clones and prunes
    Gaussians, reference controllers/clone.py:31-56, prune.py:34-45) and allocates only when a
    buffer must grow, so K changes within the capacity allocate nothing."""

    def __init__(self, out_features: int, in_features: int, k: int, device, *, tile_out: int = 16,
                 tile_in: int = 16, sigma_multiplier: float = 3.0, normalize: bool = False,
                 clamp_quad: float | None = 80.0, ids_capacity: int | None = None,
                 k_capacity: int | None = None, grads: bool = True):
        self.M, self.N = int(out_features), int(in_features)
        self.device = torch.device(device)
        self.cfg = N.make_config(tile_out, tile_in, sigma_multiplier, normalize, clamp_quad)
        L = N.lib()
        R, C = ctypes.c_int64(), ctypes.c_int64()
        N.check(L.gf_tile_grid(self.M, self.N, ctypes.byref(self.cfg), ctypes.byref(R),
                               ctypes.byref(C)), "gf_tile_grid")
        self.num_tile_rows, self.num_tile_cols = R.value, C.value
        self.T = R.value * C.value
        dev = self.device
        self.tile_ptr = torch.empty(self.T + 1, dtype=torch.int64, device=dev)
        self.num_pairs = torch.empty(1, dtype=torch.int64, device=dev)
        self.delta = torch.empty(self.M * self.N, dtype=torch.float32, device=dev)
        self._own_grads = bool(grads)
        self.K = self.k_capacity = self.capacity = 0
        self.fwd_ws_bytes = self.bwd_ws_bytes = 0
        self.fwd_ws = self.bwd_ws = self.ids = None
        self._d_mu = self._d_chol_raw = self._d_amp = None
        self.allocations = 0  # buffer (re)allocations made by resize()
        if ids_capacity is None:
            ids_capacity = int(k) * self.T  # every Gaussian on every tile
        self.resize(k, ids_capacity=ids_capacity, k_capacity=k_capacity)

    def resize(self, k: int, *, ids_capacity: int | None = None, k_capacity: int | None = None) -> bool:
        """Moves the plan to ``k`` Gaussians (and at least ``ids_capacity`` gaussian ids); the
        capacities only grow.  Returns True when a buffer was reallocated."""
        k = int(k)
        if k < 0:
            raise ValueError("k must be >= 0")
        L = N.lib()
        kc = max(k, int(k_capacity or 0), self.k_capacity)
        dev, grew = self.device, False

        def need(fn, kk):
            return int(fn(self.M, self.N, kk, ctypes.byref(self.cfg)))

        fwd = need(L.gf_forward_workspace_bytes, k)
        if self.fwd_ws is None or self.fwd_ws.numel() < fwd:
            # the largest need of any K up to the capacity (the bytes are not monotone in K)
            self.fwd_ws = torch.empty(max(fwd, need(L.gf_forward_workspace_bytes_max, kc)), dtype=torch.uint8,
                                      device=dev)
            grew = True
        bwd = need(L.gf_backward_workspace_bytes, k)
        if self.bwd_ws is None or self.bwd_ws.numel() < bwd:
            # zeroed once: every backward leaves its accumulators zero again
            self.bwd_ws = torch.zeros(max(bwd, need(L.gf_backward_workspace_bytes, kc)), dtype=torch.uint8,
                                      device=dev)
            grew = True
        ids = max(int(ids_capacity if ids_capacity is not None else self.capacity), 1)
        if self.ids is None or self.ids.numel() < ids:
            self.ids = torch.empty(ids, dtype=torch.int64, device=dev)
            grew = True
        if self._own_grads and (self._d_mu is None or self._d_mu.shape[0] < k):
            rows = max(k, kc)
            self._d_mu = torch.empty(rows, 2, dtype=torch.float32, device=dev)
            self._d_chol_raw = torch.empty(rows, 3, dtype=torch.float32, device=dev)
            self._d_amp = torch.empty(rows, 1, dtype=torch.float32, device=dev)
            grew = True
        if self._own_grads:
            self.d_mu, self.d_chol_raw, self.d_amp = self._d_mu[:k], self._d_chol_raw[:k], self._d_amp[:k]
        self.K, self.k_capacity = k, kc
        self.fwd_ws_bytes, self.bwd_ws_bytes = self.fwd_ws.numel(), self.bwd_ws.numel()
        self.capacity = self.ids.numel()
        self.allocations += int(grew)
        return grew

    def _stream(self) -> int:
        return N.stream_handle(self.device)

    # The three forward phases and two backward phases are exposed separately so that each
    # kernel can be timed on its own; forward() / backward() run them in order.
    def bin(self, mu, chol_raw, amp) -> None:
        N.check(N.lib().gf_forward_bin(ctypes.byref(self.cfg), self.M, self.N, self.K, N.ptr(mu),
                                       N.ptr(chol_raw), N.ptr(amp), self.tile_ptr.data_ptr(),
                                       self.num_pairs.data_ptr(), None, self.fwd_ws.data_ptr(),
                                       self.fwd_ws_bytes, self._stream()), "gf_forward_bin")

    def emit(self, mu, amp) -> None:
        N.check(N.lib().gf_forward_emit(ctypes.byref(self.cfg), self.M, self.N, self.K, N.ptr(mu),
                                        N.ptr(amp), self.tile_ptr.data_ptr(), self.ids.data_ptr(),
                                        self.capacity, self.fwd_ws.data_ptr(), self.fwd_ws_bytes,
                                        self._stream()),
                "gf_forward_emit")

    def render(self, row_coords, col_coords) -> torch.Tensor:
        """Renders from the Gaussian constants the last ``emit`` stored (and sorts the ids)."""
        N.check(N.lib().gf_forward_render(ctypes.byref(self.cfg), self.M, self.N, self.K,
                                          row_coords.data_ptr(), col_coords.data_ptr(),
                                          self.tile_ptr.data_ptr(), self.ids.data_ptr(), self.capacity,
                                          self.delta.data_ptr(), self.fwd_ws.data_ptr(),
                                          self.fwd_ws_bytes, self._stream()),
                "gf_forward_render")
        return self.delta

    def forward(self, row_coords, col_coords, mu, chol_raw, amp) -> torch.Tensor:
        """Bins and renders into ``self.delta`` (and ``tile_ptr`` / ``ids``); returns delta.
        One call (gf_forward) running the three phases."""
        N.check(N.lib().gf_forward(ctypes.byref(self.cfg), self.M, self.N, self.K, row_coords.data_ptr(),
                                   col_coords.data_ptr(), N.ptr(mu), N.ptr(chol_raw), N.ptr(amp),
                                   self.tile_ptr.data_ptr(), self.num_pairs.data_ptr(), self.ids.data_ptr(),
                                   self.capacity, self.delta.data_ptr(), self.fwd_ws.data_ptr(),
                                   self.fwd_ws_bytes, self._stream()), "gf_forward")
        return self.delta

    def forward_phases(self, row_coords, col_coords, mu, chol_raw, amp) -> torch.Tensor:
        """The forward as its three phases (bin, emit, render): the same outputs as forward()."""
        self.bin(mu, chol_raw, amp)
        self.emit(mu, amp)
        return self.render(row_coords, col_coords)

    def backward_reduce(self, grad, row_coords, col_coords, mu, chol_raw, num_pairs: int | None = None,
                        reuse_forward: bool = True):
        """Per-tile moments.  With ``reuse_forward`` the Gaussian constants come from the last
        forward's workspace (same mu / chol_raw), else they are recomputed from mu / chol_raw."""
        n = self.capacity if num_pairs is None else int(num_pairs)
        fwd = self.fwd_ws.data_ptr() if reuse_forward else None
        N.check(N.lib().gf_backward_reduce(ctypes.byref(self.cfg), self.M, self.N, self.K,
                                           grad.data_ptr(), row_coords.data_ptr(), col_coords.data_ptr(),
                                           N.ptr(mu), N.ptr(chol_raw), self.tile_ptr.data_ptr(), 1,
                                           self.ids.data_ptr(), 1, n, fwd, self.bwd_ws.data_ptr(),
                                           self.bwd_ws_bytes, self._stream()), "gf_backward_reduce")

    def backward_finish(self, chol_raw, amp, reuse_forward: bool = True):
        """Chain rule into ``d_mu``, ``d_chol_raw``, ``d_amp``.  With ``reuse_forward`` the
        Cholesky factors and covariances come from the last forward's workspace."""
        fwd = self.fwd_ws.data_ptr() if reuse_forward else None
        N.check(N.lib().gf_backward_finish(ctypes.byref(self.cfg), self.M, self.N, self.K,
                                           N.ptr(chol_raw), N.ptr(amp), N.ptr(self.d_mu),
                                           N.ptr(self.d_chol_raw), N.ptr(self.d_amp), fwd,
                                           self.bwd_ws.data_ptr(), self.bwd_ws_bytes, self._stream()),
                "gf_backward_finish")
        return self.d_mu, self.d_chol_raw, self.d_amp

    def backward(self, grad, row_coords, col_coords, mu, chol_raw, amp, num_pairs: int | None = None,
                 reuse_forward: bool = True):
        """Gradients into ``d_mu``, ``d_chol_raw``, ``d_amp`` from the last forward's binning."""
        self.backward_reduce(grad, row_coords, col_coords, mu, chol_raw, num_pairs, reuse_forward)
        return self.backward_finish(chol_raw, amp, reuse_forward)

    def backward_direct(self, grad, row_coords, col_coords, mu, chol_raw, amp, num_pairs: int | None = None,
                        max_span: int | None = None):
        """The backward in one launch (gf_backward_direct): the chain rule applied per tile with
        the maps the last forward stored, the gradients added into the forward workspace.
        Returns views (d_mu [K,2], d_chol_raw [K,3], d_amp [K,1]) of that workspace, strided over
        one 8-float slot per Gaussian: the next forward on this plan clears them, so copy what
        must outlive it.  The gradients are added into the slots (a second call after the same
        forward doubles them).  Fields where the one-launch kernel does not apply run the
        reduction and the finish, which adds into the same slots; so do fields whose widest
        rectangle ``max_span`` (from :meth:`bin_info`; None: not known) covers 320 tiles or more."""
        n = self.capacity if num_pairs is None else int(num_pairs)
        span = -1 if max_span is None else int(max_span)
        L = N.lib()
        N.check(L.gf_backward_direct(ctypes.byref(self.cfg), self.M, self.N, self.K, grad.data_ptr(),
                                     row_coords.data_ptr(), col_coords.data_ptr(), N.ptr(mu), N.ptr(chol_raw),
                                     N.ptr(amp), self.tile_ptr.data_ptr(), self.ids.data_ptr(), n, span,
                                     self.fwd_ws.data_ptr(), self.fwd_ws_bytes, self.bwd_ws.data_ptr(),
                                     self.bwd_ws_bytes, self._stream()), "gf_backward_direct")
        off = int(L.gf_forward_grads_offset(self.M, self.N, self.K, ctypes.byref(self.cfg)))
        slots = self.fwd_ws[off:off + 32 * self.K].view(torch.float32).view(self.K, 8)
        return slots[:, 1:3], slots[:, 3:6], slots[:, 0:1]

    def fused_supported(self, max_span: int | None = None) -> bool:
        """Whether :meth:`fwd_bwd_fused` runs the one-pass kernel for this field at the plan's id
        capacity (16x16 tiles on the mask path, fewer than 8192 tiles, sparse, no heavy tiles) and,
        if given, widest rectangle (an earlier step's :meth:`bin_info`: under 320 tiles)."""
        span = -1 if max_span is None else int(max_span)
        return bool(N.lib().gf_fwd_bwd_fused_supported(ctypes.byref(self.cfg), self.M, self.N, self.K,
                                                       self.capacity, span))

    def fwd_bwd_fused(self, row_coords, col_coords, mu, chol_raw, amp, grad, num_pairs: int | None = None,
                      max_span: int | None = None):
        """Forward and backward with dL/d(delta) given up front (gf_fwd_bwd_fused): the binning,
        then one kernel that renders delta-W and reduces ``grad`` with the same exponentials.
        Returns (delta, (d_mu, d_chol_raw, d_amp)), the gradients as :meth:`backward_direct`
        returns them (views of the forward workspace, added into slots the binning cleared).
        Fields the one-pass kernel does not take (see :meth:`fused_supported`, ``max_span`` as
        there) run :meth:`forward` + :meth:`backward_direct` (``num_pairs`` as there)."""
        if not self.fused_supported(max_span):
            self.forward(row_coords, col_coords, mu, chol_raw, amp)
            grads = self.backward_direct(grad, row_coords, col_coords, mu, chol_raw, amp, num_pairs, max_span)
            return self.delta, grads
        L = N.lib()
        N.check(L.gf_fwd_bwd_fused(ctypes.byref(self.cfg), self.M, self.N, self.K, row_coords.data_ptr(),
                                   col_coords.data_ptr(), N.ptr(mu), N.ptr(chol_raw), N.ptr(amp), grad.data_ptr(),
                                   self.tile_ptr.data_ptr(), self.num_pairs.data_ptr(), self.ids.data_ptr(),
                                   self.capacity, self.delta.data_ptr(), self.fwd_ws.data_ptr(), self.fwd_ws_bytes,
                                   self._stream()), "gf_fwd_bwd_fused")
        off = int(L.gf_forward_grads_offset(self.M, self.N, self.K, ctypes.byref(self.cfg)))
        slots = self.fwd_ws[off:off + 32 * self.K].view(torch.float32).view(self.K, 8)
        return self.delta, (slots[:, 1:3], slots[:, 3:6], slots[:, 0:1])

    def direct_launches(self, num_pairs: int | None = None, max_span: int | None = None) -> int:
        """Launches :meth:`backward_direct` makes for ``num_pairs`` (default: the id capacity) and
        ``max_span`` (None: not known): 1, or 2 where it runs the reduction and the finish."""
        n = self.capacity if num_pairs is None else int(num_pairs)
        span = -1 if max_span is None else int(max_span)
        r = int(N.lib().gf_backward_direct_launches(ctypes.byref(self.cfg), self.M, self.N, self.K, n, span))
        if r < 0:
            N.check(-r, "gf_backward_direct_launches")
        return r

    def pairs(self) -> int:
        """Pair count of the last forward (synchronises)."""
        return int(self.num_pairs.item())

    def bin_info(self) -> tuple[int, int]:
        """(P, max_span) of the last forward: its pair count and the most tiles one Gaussian's
        rectangle covers (gf_read_bin_info; synchronises)."""
        info = N.GfBinInfo()
        N.check(N.lib().gf_read_bin_info(self.fwd_ws.data_ptr(), ctypes.byref(info), self._stream()),
                "gf_read_bin_info")
        return int(info.num_pairs), int(info.max_span)

    def status(self, which: str = "forward") -> int:
        """GF_STATUS_* bits of the last forward or backward (synchronises)."""
        ws = self.fwd_ws if which == "forward" else self.bwd_ws
        st = ctypes.c_uint32(0)
        N.check(N.lib().gf_read_status(ws.data_ptr(), 0, ctypes.byref(st), self._stream()),
                "gf_read_status")
        return st.value


class FieldBatchPlan:
    """Many fields (e.g. every adapted layer of a model) rendered and differentiated together:
    each phase is one launch over all layers (``gf_batch_forward`` / ``gf_batch_backward``).

    ``layers`` is a sequence of objects with device tensors ``row_coords``, ``col_coords``,
    ``mu``, ``chol_raw``, ``amp`` and, for the backward, ``grad`` (dL/d(delta), read in place at
    every ``backward()``); a true ``mu_tanh`` attribute marks ``mu`` as GaussianLinear's mu_raw
    (the kernels take tanh and ``d_mu`` receives dL/d(mu_raw)).  The plan keeps references to them: their storage must stay put until
    the next :meth:`update`.  Each layer gets the buffers of a :class:`FieldPlan`
    (``self.plans[i]``: delta, tile_ptr, ids, pair constants, gradients).  16x16 or 32x32 tiles
    (32x32: every layer's K <= 8192).

    A layer with a ``base_weight`` attribute (its frozen fp32 weight [M, N], contiguous) gets a
    merged output, ``self.merged[i]`` [M, N] = base_weight + ``delta_scale`` * delta-W (rounded as
    torch's ``weight + delta * scale``), written by the render; its ``grad`` is then
    dL/d(merged weight) and the gradients are those through delta_scale * delta-W.  With a false
    ``keep_delta`` attribute such a layer's delta-W is not stored (``plans[i].delta`` is not
    written; the norms still are).

    ``k_capacities`` sizes each layer's buffers and the launch grids for that many Gaussians:
    after a layer's K or tensors change (densification), :meth:`update` re-plans in place, and
    for K within the capacities the launch grids and the plan buffer stay the same, so
    launches captured in a graph remain valid.
    """

    def __init__(self, layers, device, *, capacities, k_capacities=None, tile_out: int = 16,
                 tile_in: int = 16, sigma_multiplier: float = 3.0, normalize: bool = False,
                 clamp_quad: float | None = 80.0):
        self.device = torch.device(device)
        self.cfg = N.make_config(tile_out, tile_in, sigma_multiplier, normalize, clamp_quad)
        self._plan_kwargs = dict(tile_out=tile_out, tile_in=tile_in, sigma_multiplier=sigma_multiplier,
                                 normalize=normalize, clamp_quad=clamp_quad)
        self.plans: list[FieldPlan] = []
        self.merged: list[torch.Tensor | None] = []
        self.plan = None
        self.info = None
        self.grad_flat = None
        self.update(layers, capacities=capacities, k_capacities=k_capacities)

    def update(self, layers=None, *, capacities=None, k_capacities=None) -> bool:
        """Re-plans for ``layers`` (default: the current ones, re-read): each layer's K and
        tensors, with at least ``capacities`` gaussian ids and ``k_capacities`` Gaussians per
        layer.  Buffers grow only when they must.  Returns True when the launch grids and the
        plan buffer are unchanged (graphs captured over forward() / backward() stay valid: the
        kernels read every layer's buffers from the plan).  ``self.reallocated`` tells whether a
        layer buffer or the gradient buffer had to grow.  Synchronises the stream (the plan is
        uploaded from host memory)."""
        if layers is not None:
            layers = list(layers)
            if self.plans and len(layers) != len(self.plans):
                raise ValueError(f"expected {len(self.plans)} layers, got {len(layers)}")
            self.layers = layers
        n = len(self.layers)
        caps = list(capacities) if capacities is not None else [None] * n
        kcs = list(k_capacities) if k_capacities is not None else [None] * n
        if len(caps) != n or len(kcs) != n:
            raise ValueError("capacities / k_capacities need one entry per layer")
        grew = False
        for i, ly in enumerate(self.layers):
            M, Nf, K = int(ly.row_coords.numel()), int(ly.col_coords.numel()), int(ly.mu.shape[0])
            if i < len(self.plans):
                pl = self.plans[i]
                if (pl.M, pl.N) != (M, Nf):
                    raise ValueError(f"layer {i}: shape {M}x{Nf} differs from the planned {pl.M}x{pl.N}")
                grew |= pl.resize(K, ids_capacity=caps[i], k_capacity=kcs[i])
            else:
                self.plans.append(FieldPlan(M, Nf, K, self.device, ids_capacity=caps[i],
                                            k_capacity=kcs[i], grads=False, **self._plan_kwargs))
        # Every layer's gradients in one buffer (per layer: d_mu [K,2], d_chol_raw [K,3],
        # d_amp [K,1]), so that they can be copied out with one launch.
        self.grad_numel = sum(6 * pl.K for pl in self.plans)
        if self.grad_flat is None or self.grad_flat.numel() < self.grad_numel:
            grew = grew or self.grad_flat is not None
            self.grad_flat = torch.empty(max(sum(6 * pl.k_capacity for pl in self.plans), 1),
                                         dtype=torch.float32, device=self.device)
        o = 0
        for pl in self.plans:
            K = pl.K
            pl.d_mu = self.grad_flat[o:o + 2 * K].view(K, 2)
            pl.d_chol_raw = self.grad_flat[o + 2 * K:o + 5 * K].view(K, 3)
            pl.d_amp = self.grad_flat[o + 5 * K:o + 6 * K].view(K, 1)
            o += 6 * K
        while len(self.merged) < n:
            self.merged.append(None)
        table = (N.GfLayer * max(n, 1))()
        for i, (ly, pl) in enumerate(zip(self.layers, self.plans)):
            grad = getattr(ly, "grad", None)
            base = getattr(ly, "base_weight", None)
            merged, scale, keep = None, 1.0, True
            if base is not None:
                if (base.dtype != torch.float32 or not base.is_contiguous() or base.numel() != pl.M * pl.N
                        or base.device != self.device):
                    raise ValueError(f"layer {i}: base_weight must be a contiguous float32 tensor of "
                                     f"{pl.M}x{pl.N} elements on {self.device}")
                merged = self.merged[i]
                if merged is None or merged.numel() != pl.M * pl.N:
                    grew = grew or merged is not None
                    merged = torch.empty(pl.M, pl.N, dtype=torch.float32, device=self.device)
                scale = float(getattr(ly, "delta_scale", 1.0))
                keep = bool(getattr(ly, "keep_delta", True))
            self.merged[i] = merged
            table[i] = N.GfLayer(
                pl.M, pl.N, pl.K, ly.row_coords.data_ptr(), ly.col_coords.data_ptr(), N.ptr(ly.mu),
                N.ptr(ly.chol_raw), N.ptr(ly.amp), pl.delta.data_ptr() if keep else None, pl.tile_ptr.data_ptr(),
                pl.num_pairs.data_ptr(), pl.ids.data_ptr(), pl.capacity,
                pl.fwd_ws.data_ptr(), pl.fwd_ws_bytes, None if grad is None else grad.data_ptr(),
                N.ptr(pl.d_mu), N.ptr(pl.d_chol_raw), N.ptr(pl.d_amp), pl.bwd_ws.data_ptr(),
                pl.bwd_ws_bytes, pl.k_capacity, 1 if getattr(ly, "mu_tanh", False) else 0, 0,
                None if base is None else base.data_ptr(), None if merged is None else merged.data_ptr(),
                scale, 0)
        self.reallocated = grew
        info = N.GfBatchInfo()
        L = N.lib()
        N.check(L.gf_batch_plan(ctypes.byref(self.cfg), table, n, None, 0, ctypes.byref(info),
                                self._stream()), "gf_batch_plan (size)")
        old, old_plan = self.info, self.plan
        if self.plan is None or self.plan.numel() < int(info.plan_bytes):
            self.plan = torch.empty(max(int(info.plan_bytes), 256), dtype=torch.uint8, device=self.device)
        N.check(L.gf_batch_plan(ctypes.byref(self.cfg), table, n, self.plan.data_ptr(), self.plan.numel(),
                                ctypes.byref(info), self._stream()), "gf_batch_plan")
        self.info = info
        self._grads = None
        return (old is not None and self.plan is old_plan and
                (old.tile_blocks, old.emit_blocks, old.finish_blocks, old.render_blocks, old.tile_render) ==
                (info.tile_blocks, info.emit_blocks, info.finish_blocks, info.render_blocks, info.tile_render))

    def _stream(self) -> int:
        return N.stream_handle(self.device)

    def forward(self, phases: int = N.GF_PHASE_ALL) -> None:
        N.check(N.lib().gf_batch_forward(self.plan.data_ptr(), ctypes.byref(self.info), phases,
                                         self._stream()), "gf_batch_forward")

    def backward(self, phases: int = N.GF_PHASE_ALL) -> None:
        N.check(N.lib().gf_batch_backward(self.plan.data_ptr(), ctypes.byref(self.info), phases,
                                          self._stream()), "gf_batch_backward")

    def set_grads(self, grads, check: bool = True) -> None:
        """dL/d(delta) of every layer for the next ``backward()`` (contiguous fp32 device tensors
        of M*N elements, kept alive by the plan until replaced); no host synchronisation.
        ``check=False`` skips the per-tensor checks for callers that guarantee them."""
        grads = list(grads)
        if len(grads) != len(self.plans):
            raise ValueError(f"expected {len(self.plans)} gradients, got {len(grads)}")
        for i, (g, pl) in enumerate(zip(grads, self.plans) if check else ()):
            if (g.dtype != torch.float32 or not g.is_contiguous() or g.numel() != pl.M * pl.N
                    or g.device != self.device):
                raise ValueError(f"layer {i}: dL/d(delta) must be a contiguous float32 tensor of "
                                 f"{pl.M * pl.N} elements on {self.device}")
        ptrs = (ctypes.c_void_p * max(len(grads), 1))(*[g.data_ptr() for g in grads])
        N.check(N.lib().gf_batch_set_grads(self.plan.data_ptr(), ctypes.byref(self.info), ptrs,
                                           self._stream()), "gf_batch_set_grads")
        self._grads = grads

    def read(self, clear: bool = False, norms: bool = False):
        """(GF_STATUS_* bits, pair count) of every layer's last pass -- plus, with ``norms``, the
        Frobenius norm of every layer's delta-W from the last forward -- in one read-back
        (synchronises)."""
        n = len(self.plans)
        st = (ctypes.c_uint32 * max(n, 1))()
        pairs = (ctypes.c_int64 * max(n, 1))()
        nrm = (ctypes.c_double * max(n, 1))()
        N.check(N.lib().gf_batch_read(self.plan.data_ptr(), ctypes.byref(self.info), 1 if clear else 0, st,
                                      pairs, nrm if norms else None, self._stream()), "gf_batch_read")
        out = ([int(st[i]) for i in range(n)], [int(pairs[i]) for i in range(n)])
        return out + ([float(nrm[i]) for i in range(n)],) if norms else out

    def status(self) -> list[int]:
        """Forward | backward GF_STATUS_* bits per layer (synchronises)."""
        return self.read()[0]


class StaticFieldPlan:
    """One field whose forward and one-launch backward can be captured in a HIP graph once and
    replayed across changes of K (gf_forward_kcap / gf_backward_direct_kcap).

    Densification clones and prunes Gaussians every 50-200 steps (reference
    controllers/clone.py:31-56, prune.py:34-45), which gives the parameters another K.  Here
    everything a launch depends on is fixed by ``k_capacity``: the plan owns the parameter buffers
    (``mu`` [k_capacity, 2], ``chol_raw`` [k_capacity, 3], ``amp`` [k_capacity, 1]) and the device K
    (``k_dev``), and the kernels read the live K and pair count from device memory.
    :meth:`set_params` copies a new parameter set in (any K up to the capacity) and writes K, on
    the current stream and outside any capture; a graph captured over :meth:`forward` and
    :meth:`backward_direct` then replays with the new field and no re-capture.

    The mask path only: 16x16 or 32x32 tiles, 1 <= k_capacity <= 8192.  ``ids_capacity`` bounds the
    pairs of every K the plan will see (past it GF_STATUS_CAPACITY is set: check :meth:`status`).
    """

    def __init__(self, out_features: int, in_features: int, k_capacity: int, device, *, ids_capacity: int,
                 tile_out: int = 16, tile_in: int = 16, sigma_multiplier: float = 3.0, normalize: bool = False,
                 clamp_quad: float | None = 80.0):
        kc = int(k_capacity)
        # workspaces, tile_ptr, ids and delta of a FieldPlan laid out for the capacity
        self.buffers = FieldPlan(out_features, in_features, kc, device, tile_out=tile_out, tile_in=tile_in,
                                 sigma_multiplier=sigma_multiplier, normalize=normalize, clamp_quad=clamp_quad,
                                 ids_capacity=ids_capacity, grads=False)
        b = self.buffers
        self.M, self.N, self.k_capacity, self.device, self.cfg = b.M, b.N, kc, b.device, b.cfg
        self.mu = torch.zeros(kc, 2, dtype=torch.float32, device=self.device)
        self.chol_raw = torch.zeros(kc, 3, dtype=torch.float32, device=self.device)
        self.amp = torch.zeros(kc, 1, dtype=torch.float32, device=self.device)
        self.k_dev = torch.zeros(1, dtype=torch.int64, device=self.device)
        self.live_k = 0

    @property
    def delta(self) -> torch.Tensor:
        return self.buffers.delta

    @property
    def tile_ptr(self) -> torch.Tensor:
        return self.buffers.tile_ptr

    @property
    def ids(self) -> torch.Tensor:
        return self.buffers.ids

    def set_params(self, mu, chol_raw, amp) -> None:
        """The field's Gaussians for the next forward: K = mu.shape[0] <= k_capacity rows of
        mu [K, 2], chol_raw [K, 3], amp [K, 1] (fp32, on the plan's device), copied in on the current
        stream; the capacity's other rows are left as they are (the kernels read only K rows)."""
        k = int(mu.shape[0])
        if not (0 <= k <= self.k_capacity):
            raise ValueError(f"K = {k} outside [0, {self.k_capacity}] (the plan's capacity)")
        if tuple(chol_raw.shape) != (k, 3) or tuple(amp.shape) != (k, 1) or tuple(mu.shape) != (k, 2):
            raise ValueError("mu / chol_raw / amp must have shapes [K,2], [K,3], [K,1]")
        with torch.no_grad():
            self.mu[:k].copy_(mu)
            self.chol_raw[:k].copy_(chol_raw)
            self.amp[:k].copy_(amp)
            self.k_dev.fill_(k)
        self.live_k = k

    def forward(self, row_coords, col_coords) -> torch.Tensor:
        """Bins and renders the current parameters into ``delta`` (and tile_ptr, the ids, P)."""
        b = self.buffers
        N.check(N.lib().gf_forward_kcap(ctypes.byref(self.cfg), self.M, self.N, self.k_capacity, self.k_dev.data_ptr(),
                                        row_coords.data_ptr(), col_coords.data_ptr(), self.mu.data_ptr(),
                                        self.chol_raw.data_ptr(), self.amp.data_ptr(), b.tile_ptr.data_ptr(),
                                        b.num_pairs.data_ptr(), b.ids.data_ptr(), b.capacity, b.delta.data_ptr(),
                                        b.fwd_ws.data_ptr(), b.fwd_ws_bytes, b._stream()), "gf_forward_kcap")
        return b.delta

    def backward_direct(self, grad, row_coords, col_coords):
        """The gradients of the last forward's field into the forward workspace's slots (as
        FieldPlan.backward_direct: added into slots the forward cleared); returns views
        (d_mu, d_chol_raw, d_amp) of the slots of the capacity: rows 0 .. live_k - 1 are the field's."""
        b = self.buffers
        N.check(N.lib().gf_backward_direct_kcap(
            ctypes.byref(self.cfg), self.M, self.N, self.k_capacity, self.k_dev.data_ptr(), grad.data_ptr(),
            row_coords.data_ptr(), col_coords.data_ptr(), self.mu.data_ptr(), self.chol_raw.data_ptr(),
            self.amp.data_ptr(), b.tile_ptr.data_ptr(), b.ids.data_ptr(), b.num_pairs.data_ptr(), b.capacity,
            b.fwd_ws.data_ptr(), b.fwd_ws_bytes, b.bwd_ws.data_ptr(), b.bwd_ws_bytes, b._stream()),
            "gf_backward_direct_kcap")
        off = int(N.lib().gf_forward_grads_offset(self.M, self.N, self.k_capacity, ctypes.byref(self.cfg)))
        slots = b.fwd_ws[off:off + 32 * self.k_capacity].view(torch.float32).view(self.k_capacity, 8)
        return slots[:, 1:3], slots[:, 3:6], slots[:, 0:1]

    def direct_launches(self) -> int:
        """Launches :meth:`backward_direct` makes (1, or 2 for reduction + finish), the same for every K."""
        r = int(N.lib().gf_backward_direct_launches(ctypes.byref(self.cfg), self.M, self.N, self.k_capacity,
                                                    self.buffers.capacity, -1))
        if r < 0:
            N.check(-r, "gf_backward_direct_launches")
        return r

    def pairs(self) -> int:
        """Pair count of the last forward (synchronises)."""
        return self.buffers.pairs()

    def status(self, which: str = "forward") -> int:
        """GF_STATUS_* bits of the last forward or backward (synchronises)."""
        return self.buffers.status(which)
