"""The adapted linear layer's use of the Gaussian-field path, on the MI355X runtime.

``GaussianLinear`` has the surface of the reference layer (gaussian_peft/layers/gaussian_linear.py
:19-280) for the two execution modes that run the field path:

* ``cuda_field_train``             ``gaussian_field_train`` (autograd through the gfx950 kernels)
* ``cuda_field_stage2_validation`` forward-only with the binning metadata

``compute_delta_weight`` (gaussian_linear.py:162-220) takes mu = tanh(mu_raw), renders the field
with the quadratic form clamped at 80, reshapes it to [out_features, in_features], records
``delta_w_norm`` in ``last_forward_metadata`` and scales by ``adapter_scale``.  ``forward`` adds
x @ delta-W^T to the frozen base linear in row chunks of the output (gaussian_linear.py:222-253).

The reference layer itself runs unchanged on ``guass_amd.cuda_field`` (it imports only
``gaussian_field_train`` and ``gaussian_field_cuda_field_stage2_validation`` from the runtime);
this module serves users of this package that do not carry the reference.  Parameter
initialisation supports ``uniform_grid`` and ``random_uniform`` (gaussian_linear.py:104-129);
``grid_overlap`` belongs to the reference's initialiser package and is not built here -- load its
parameters with ``load_adapter_state``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from guass_amd.cuda_field.runtime import (
    gaussian_field_cuda_field_stage2_validation,
    gaussian_field_train,
)

FIELD_EXECUTION_MODES = ("cuda_field_train", "cuda_field_stage2_validation")
_MODE_ALIASES = {"cuda_field_stage3_custom": "cuda_field_train"}  # config/adapter.py:82-90
CLAMP_QUAD = 80.0  # what the layer passes to the field (gaussian_linear.py:176,190)


@dataclass(slots=True)
class GaussianAdapterConfig:
    """Adapter configuration (field names and defaults of config/adapter.py:8-29)."""

    init_num_gaussians: int = 32
    init_method: str = "random_uniform"
    coord_norm: str = "minus_one_to_one"
    covariance_type: str = "cholesky"
    use_amp_scaling: bool = True
    adapter_scale: float = 1.0
    chunk_size: int | None = None
    train_bias: bool = False
    merge_weights: bool = False
    normalize_gaussian: bool = False
    compute_dtype: torch.dtype = torch.float32
    eps: float = 1e-5
    init_amp_scale: float = 1e-4
    init_chol_scale_multiplier: float = 1.5
    min_cov_diag: float = 1e-4
    execution_mode: str = "cuda_field_train"
    tile_out: int = 32
    tile_in: int = 32
    sigma_multiplier: float = 3.0
    # How forward composes the base linear with delta-W (no counterpart field in the reference,
    # whose layer always does "row_chunk", gaussian_linear.py:222-253): "merged" runs one GEMM on
    # W + delta-W instead of the base GEMM plus row-chunked delta GEMMs and an output clone.
    delta_apply: str = "row_chunk"

    def validate(self) -> None:
        """The checks of config/adapter.py:31-79 that concern the field path."""
        if self.init_num_gaussians <= 0:
            raise ValueError("init_num_gaussians must be positive")
        if self.init_method not in ("uniform_grid", "random_uniform", "grid_overlap"):
            raise ValueError(f"Unsupported init_method={self.init_method!r}.")
        if self.coord_norm != "minus_one_to_one":
            raise ValueError(f"Unsupported coord_norm={self.coord_norm!r}.")
        if self.covariance_type != "cholesky":
            raise ValueError(f"Unsupported covariance_type={self.covariance_type!r}.")
        if self.eps <= 0:
            raise ValueError("eps must be positive")
        if self.min_cov_diag <= 0:
            raise ValueError("min_cov_diag must be positive")
        if self.init_amp_scale < 0:
            raise ValueError("init_amp_scale must be non-negative")
        if self.init_chol_scale_multiplier <= 0:
            raise ValueError("init_chol_scale_multiplier must be positive")
        if self.tile_out <= 0 or self.tile_in <= 0:
            raise ValueError("tile_out and tile_in must be positive")
        if self.sigma_multiplier <= 0:
            raise ValueError("sigma_multiplier must be positive")
        if self.delta_apply not in ("row_chunk", "merged"):
            raise ValueError(f"Unsupported delta_apply={self.delta_apply!r}.")
        if self.merge_weights:
            raise ValueError("merge_weights is disabled in the first implementation")
        self.execution_mode = _MODE_ALIASES.get(self.execution_mode, self.execution_mode)
        if self.execution_mode not in FIELD_EXECUTION_MODES:
            raise ValueError(
                f"execution_mode={self.execution_mode!r} is not a Gaussian-field mode; this "
                f"package runs {FIELD_EXECUTION_MODES}")


class GaussianLinear(nn.Linear):
    """nn.Linear with a frozen base weight plus a Gaussian-field delta-W."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, *,
                 adapter_config: GaussianAdapterConfig, device=None, dtype=None) -> None:
        super().__init__(in_features, out_features, bias=bias, device=device, dtype=dtype)
        adapter_config.validate()
        self.adapter_config = adapter_config
        self.merged = False
        self.weight.requires_grad = False
        if self.bias is not None and not adapter_config.train_bias:
            self.bias.requires_grad = False
        # linspace(-1, 1) axes on the layer's device (kernels/coords.py:23-34)
        self.register_buffer("row_coords", torch.linspace(-1.0, 1.0, out_features, device=self.weight.device),
                             persistent=False)
        self.register_buffer("col_coords", torch.linspace(-1.0, 1.0, in_features, device=self.weight.device),
                             persistent=False)
        self.last_forward_metadata: dict = {}
        # from GaussianFieldBatch.render(): (tensor, norm of delta-W, kind), kind "delta" (delta-W) or
        # "merged_weight" (weight + adapter_scale * delta-W, for delta_apply "merged")
        self._batched_delta: tuple[Tensor, float, str] | None = None
        self.reset_gaussian_parameters()

    @classmethod
    def from_linear(cls, linear: nn.Linear, adapter_config: GaussianAdapterConfig) -> "GaussianLinear":
        layer = cls(linear.in_features, linear.out_features, bias=linear.bias is not None,
                    adapter_config=adapter_config, device=linear.weight.device,
                    dtype=linear.weight.dtype)
        with torch.no_grad():
            layer.weight.copy_(linear.weight)
            if linear.bias is not None:
                layer.bias.copy_(linear.bias)
        return layer

    @property
    def num_gaussians(self) -> int:
        return int(self.mu_raw.shape[0])

    # ---------------------------------------------------------------- parameters

    def _parameter_dtype(self) -> torch.dtype:
        dt = self.adapter_config.compute_dtype
        return torch.float32 if dt in (torch.float16, torch.bfloat16) else dt

    def reset_gaussian_parameters(self) -> None:
        """uniform_grid / random_uniform initialisation (gaussian_linear.py:104-138)."""
        cfg = self.adapter_config
        if cfg.init_method == "grid_overlap":
            raise NotImplementedError(
                "init_method='grid_overlap' uses the reference's initialiser package, which is "
                "not part of this build; initialise elsewhere and call load_adapter_state()")
        k, dev, dt = cfg.init_num_gaussians, self.weight.device, self._parameter_dtype()
        if cfg.init_method == "uniform_grid":
            side = math.ceil(math.sqrt(k))
            ax = torch.linspace(-1.0, 1.0, side, device=dev, dtype=dt)
            gx, gy = torch.meshgrid(ax, ax, indexing="ij")
            mu = torch.stack((gx, gy), dim=-1).reshape(-1, 2)[:k]
        else:
            mu = torch.empty(k, 2, device=dev, dtype=dt).uniform_(-1.0, 1.0)
        scale = max(2.0 / math.sqrt(max(k, 1)) * cfg.init_chol_scale_multiplier, cfg.min_cov_diag ** 0.5)
        chol_raw = torch.zeros(k, 3, device=dev, dtype=dt)
        # inverse softplus in the parameter dtype on the layer's device, as the reference
        # computes it (gaussian_linear.py:115-125,286-288); a float64 evaluation rounded once
        # differs from it by an ulp for some K
        target_diag = torch.full((k, 2), scale, device=dev, dtype=dt)
        chol_raw[:, 0] = torch.log(torch.expm1(target_diag[:, 0] - cfg.eps))
        chol_raw[:, 2] = torch.log(torch.expm1(target_diag[:, 1] - cfg.eps))
        amp = torch.zeros(k, 1, device=dev, dtype=dt)
        if cfg.init_amp_scale > 0:
            amp.normal_(mean=0.0, std=cfg.init_amp_scale)
        self.mu_raw = nn.Parameter(torch.atanh(mu.clamp(-0.999999, 0.999999)))
        self.chol_raw = nn.Parameter(chol_raw)
        self.amp = nn.Parameter(amp)

    def get_gaussian_parameters(self) -> dict[str, nn.Parameter]:
        return {"mu_raw": self.mu_raw, "chol_raw": self.chol_raw, "amp": self.amp}

    def get_adapter_state(self) -> dict[str, Tensor]:
        return {k: v.detach().clone() for k, v in self.get_gaussian_parameters().items()}

    def load_adapter_state(self, state: dict[str, Tensor]) -> None:
        self.replace_gaussian_parameters_(mu_raw=state["mu_raw"], chol_raw=state["chol_raw"],
                                          amp=state["amp"])

    def replace_gaussian_parameters_(self, *, mu_raw: Tensor | None = None,
                                     chol_raw: Tensor | None = None, amp: Tensor | None = None) -> None:
        dev, dt = self.weight.device, self._parameter_dtype()
        if mu_raw is not None:
            self.mu_raw = nn.Parameter(mu_raw.to(device=dev, dtype=dt))
        if chol_raw is not None:
            self.chol_raw = nn.Parameter(chol_raw.to(device=dev, dtype=dt))
        if amp is not None:
            self.amp = nn.Parameter(amp.to(device=dev, dtype=dt))

    def materialize_mu(self) -> Tensor:
        return torch.tanh(self.mu_raw)

    # ---------------------------------------------------------------- delta-W

    def compute_delta_weight(self) -> Tensor:
        cfg = self.adapter_config
        pending = self._batched_delta
        if pending is not None and pending[2] == "delta":
            # rendered for this step by GaussianFieldBatch.render(), with its norm from the
            # batch's one read-back (no per-layer synchronisation); used once
            self._batched_delta = None
            delta_weight, norm, _ = pending
            metadata = {"execution_mode": cfg.execution_mode, "accumulate_backend": "batched_fields",
                        "delta_w_norm": norm}
            self.last_forward_metadata = metadata
            return delta_weight * cfg.adapter_scale
        ctx = torch.autocast(device_type="cuda", enabled=False) if self.weight.is_cuda else _null()
        with ctx:
            kwargs = dict(row_coords=self.row_coords, col_coords=self.col_coords,
                          mu=self.materialize_mu().contiguous(), chol_raw=self.chol_raw,
                          amp=self.amp, tile_out=cfg.tile_out, tile_in=cfg.tile_in,
                          sigma_multiplier=cfg.sigma_multiplier, normalize=cfg.normalize_gaussian,
                          clamp_quad=CLAMP_QUAD)
            if cfg.execution_mode == "cuda_field_stage2_validation":
                delta, metadata = gaussian_field_cuda_field_stage2_validation(**kwargs)
            else:
                delta = gaussian_field_train(**kwargs)
                metadata = {"execution_mode": "cuda_field_train",
                            "accumulate_backend": "cuda_field_train"}
        delta_weight = delta.reshape(self.out_features, self.in_features)
        metadata = dict(metadata)
        metadata["delta_w_norm"] = float(delta_weight.detach().float().norm().item())
        self.last_forward_metadata = metadata
        return delta_weight * cfg.adapter_scale

    def _delta_apply_row_chunk(self) -> int:
        return min(self.out_features, max(max(1, int(self.adapter_config.tile_out)), 64))

    def forward(self, input: Tensor) -> Tensor:
        pending = self._batched_delta
        if pending is not None and pending[2] == "merged_weight":
            # weight + adapter_scale * delta-W, written by GaussianFieldBatch's render (the same
            # fp32 roundings as the two elementwise operations below); used once.  (Plain
            # attributes, set without nn.Module's bookkeeping: this runs per layer per step.)
            merged, norm, _ = pending
            self.__dict__["_batched_delta"] = None
            self.__dict__["last_forward_metadata"] = {
                "execution_mode": self.adapter_config.execution_mode, "accumulate_backend": "batched_fields",
                "delta_w_norm": norm, "linear_composition": "merged_weight"}
            return F.linear(input, merged, self._parameters["bias"])
        delta_weight = self.compute_delta_weight().to(dtype=self.weight.dtype)
        if self.adapter_config.delta_apply == "merged":
            metadata = dict(self.last_forward_metadata)
            metadata["linear_composition"] = "merged_weight"
            self.last_forward_metadata = metadata
            return F.linear(input, self.weight + delta_weight, self.bias)
        base = F.linear(input, self.weight, self.bias)
        chunk = self._delta_apply_row_chunk()
        metadata = dict(self.last_forward_metadata)
        metadata["linear_composition"] = "base_plus_delta_row_chunk_accumulate"
        metadata["delta_apply_row_chunk"] = float(chunk)
        self.last_forward_metadata = metadata
        out = base.clone()
        for r0 in range(0, self.out_features, chunk):
            r1 = min(r0 + chunk, self.out_features)
            out[..., r0:r1].add_(F.linear(input, delta_weight[r0:r1, :], None))
        return out


class _null:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


class _BatchedFieldFunction(torch.autograd.Function):
    """Autograd node of GaussianFieldBatch.render(): inputs (mu_raw, chol_raw, amp) of every
    layer, outputs every layer's delta-W [out_features, in_features].  The batched kernels take
    mu = tanh(mu_raw) (gaussian_linear.py:153-154) themselves and return dL/d(mu_raw)."""

    @staticmethod
    def forward(ctx, fb: "GaussianFieldBatch", *params: Tensor):
        ctx.fb = fb
        return tuple(fb._run_forward())

    @staticmethod
    def backward(ctx, *grads: Tensor):
        fb: GaussianFieldBatch = ctx.fb
        return (None, *fb._run_backward(grads))


class GaussianFieldBatch:
    """The delta-W of many GaussianLinear layers rendered together: one launch per forward phase
    for all layers at the start of a step, and one launch per backward phase for all their
    dL/d(delta-W) (the reference renders each layer inside its own forward,
    gaussian_linear.py:178-190).

    Per training step::

        fb = GaussianFieldBatch(layers)   # once
        fb.render()                       # step start: every layer's delta-W, with autograd
        loss = model(x); loss.backward()  # each layer's forward uses its rendered delta-W once

    A layer whose forward does not run in the step contributes a zero dL/d(delta-W).  The
    rendered delta-W tensors are the plan's own buffers: they hold until the next render().

    A layer with ``delta_apply="merged"`` and a contiguous fp32 weight gets weight +
    adapter_scale * delta-W from the render itself (rounded as the layer's own two elementwise
    operations would round it), and its forward is one GEMM on it; its delta-W is not stored, and
    the backward takes dL/d(merged weight) with adapter_scale applied in the chain rule.  Such a
    step makes no elementwise launches around the field kernels.
    The forward reads back every layer's status, pair count and ||delta-W|| (the layer's
    ``delta_w_norm`` metadata) at once: one host synchronisation per step, where the reference
    synchronises per layer (gaussian_linear.py:218).  A pair count past a layer's id capacity
    grows the capacities and renders again.  All layers must share the tile shape
    (16x16 or 32x32: the batched kernels), sigma multiplier and normalisation.

    ``render(check=False)`` skips the read-back: the step then makes no host synchronisation
    and no library call other than the three batched launches (forward, the gradient pointers,
    backward).  It needs the plan of an earlier checked render (the same parameter tensors and K,
    id capacities that held); ``check()`` then reads back every layer's status, pair count and
    norm once and raises if a layer's pairs passed its id capacity (a checked render() grows
    them).  The batched kernels themselves capture and replay in a HIP graph
    (``FieldBatchPlan.forward`` / ``backward``); capturing a whole step, with autograd and the
    layers' GEMMs around them, is not supported: one such capture ended the process in the HIP
    runtime's capture_end, with no cause found in this package's calls.

    Densification (the reference trainer's clone / prune, base_trainer.py:126-220) replaces a
    layer's Gaussian parameters with tensors of another K; the next render() re-plans in place.
    ``k_capacity`` (an int for every layer, or one per layer; e.g. the densify config's
    ``max_gaussians_per_layer``) sizes the buffers so that K changes up to it allocate nothing;
    past it a layer's capacity doubles.
    """

    def __init__(self, layers, *, headroom: float = 1.25, k_capacity=None):
        from guass_amd import _native as Nat

        self._Nat = Nat
        self.layers = list(layers)
        if not self.layers:
            raise ValueError("GaussianFieldBatch needs at least one layer")
        for i, ly in enumerate(self.layers):
            if not isinstance(ly, GaussianLinear):
                raise TypeError(f"layer {i} is not a GaussianLinear")
        cfgs = [ly.adapter_config for ly in self.layers]
        c0 = cfgs[0]
        for i, c in enumerate(cfgs):
            if (c.tile_out, c.tile_in) not in ((16, 16), (32, 32)):
                raise ValueError(f"layer {i}: batched fields need 16x16 or 32x32 tiles "
                                 f"(got {c.tile_out}x{c.tile_in})")
            if (c.tile_out != c0.tile_out or c.sigma_multiplier != c0.sigma_multiplier
                    or c.normalize_gaussian != c0.normalize_gaussian):
                raise ValueError(f"layer {i}: tile shape / sigma_multiplier / normalize_gaussian differ "
                                 "from layer 0")
        self.device = self.layers[0].weight.device
        if any(ly.weight.device != self.device for ly in self.layers):
            raise ValueError("all layers must live on one device")
        self.headroom = float(headroom)
        self._plan = None
        self._key = None
        self._caps = [ly.num_gaussians * 32 for ly in self.layers]  # grown from the read-back
        if k_capacity is None or isinstance(k_capacity, int):
            kc = [max(int(k_capacity or 0), ly.num_gaussians) for ly in self.layers]
        else:
            kc = [max(int(c), ly.num_gaussians) for c, ly in zip(k_capacity, self.layers, strict=True)]
        self._kcaps = kc
        self._ks = [ly.num_gaussians for ly in self.layers]
        self._pairs = None
        self._zero_grads: dict[int, Tensor] = {}
        self._norms: list[float] = []
        self._check = True  # the next forward reads back (render(check=...))
        self.replans = 0  # re-plans after the first plan (parameter tensors or K changed)

    # ---------------------------------------------------------------- plan

    @staticmethod
    def _merges(ly: "GaussianLinear") -> bool:
        """The layer takes weight + adapter_scale * delta-W from the render."""
        w = ly._parameters["weight"]
        return (ly.adapter_config.delta_apply == "merged" and w.dtype == torch.float32 and w.is_contiguous()
                and not w.requires_grad)

    def _param_key(self):
        """What the plan depends on, per layer: K, the parameter tensors' storage, and for a merging
        layer its weight's storage and adapter_scale (read through the modules' parameter dicts:
        this runs at every render)."""
        key = []
        for ly in self.layers:
            prm, cfg = ly._parameters, ly.adapter_config
            mu = prm["mu_raw"]
            merges = cfg.delta_apply == "merged"
            key.append((mu.shape[0], mu.data_ptr(), prm["chol_raw"].data_ptr(), prm["amp"].data_ptr(),
                        prm["weight"].data_ptr() if merges else 0, cfg.adapter_scale if merges else 0.0))
        return tuple(key)

    def _build(self) -> None:
        """Plans, or re-plans in place, for the layers' current K and parameter tensors (which
        the kernels read in place: mu_raw, chol_raw and amp as contiguous float32)."""
        from guass_amd.ops import FieldBatchPlan

        class _View:
            pass

        views = []
        for i, ly in enumerate(self.layers):
            for name in ("mu_raw", "chol_raw", "amp"):
                t = getattr(ly, name)
                if t.dtype != torch.float32 or not t.is_contiguous():
                    raise ValueError(f"layer {i}: {name} must be contiguous float32")
            K = ly.num_gaussians
            if K > self._kcaps[i]:
                self._kcaps[i] = max(K, 2 * self._kcaps[i])
            if K != self._ks[i] and self._pairs is not None and self._ks[i] > 0:
                # pairs scale with K: grow the id capacity with it rather than by a retry
                self._caps[i] = max(self._caps[i], int(self._pairs[i] * K / self._ks[i] * self.headroom) + 1)
            self._ks[i] = K
            v = _View()
            v.row_coords, v.col_coords = ly.row_coords, ly.col_coords
            v.mu, v.chol_raw, v.amp = ly.mu_raw, ly.chol_raw, ly.amp
            v.mu_tanh = True
            v.grad = None
            if self._merges(ly):
                v.base_weight = ly.weight.detach()
                v.delta_scale = float(ly.adapter_config.adapter_scale)
                v.keep_delta = False
            views.append(v)
        if self._plan is None:
            c0 = self.layers[0].adapter_config
            self._plan = FieldBatchPlan(views, self.device, capacities=self._caps, k_capacities=self._kcaps,
                                        tile_out=c0.tile_out, tile_in=c0.tile_in,
                                        sigma_multiplier=c0.sigma_multiplier,
                                        normalize=c0.normalize_gaussian, clamp_quad=CLAMP_QUAD)
        else:
            self._plan.update(views, capacities=self._caps, k_capacities=self._kcaps)
            self.replans += 1
        pl = self._plan
        # per layer: the merged weight where the layer merges, else delta-W
        self._kinds = ["merged_weight" if m is not None else "delta" for m in pl.merged]
        self._deltas = [m if m is not None else q.delta.view(q.M, q.N) for q, m in zip(pl.plans, pl.merged)]
        # the gradient buffer split per parameter: d_mu_raw [K,2], d_chol_raw [K,3], d_amp [K,1],
        # described by empty tensors of those shapes (one unflatten call makes all the views)
        self._grad_like = [torch.empty(sh, dtype=torch.float32, device="meta")
                           for q in pl.plans for sh in ((q.K, 2), (q.K, 3), (q.K, 1))]
        self._key = self._param_key()

    # ---------------------------------------------------------------- passes

    def render(self, check: bool = True) -> list[Tensor]:
        """Renders every layer's delta-W for this step (autograd-tracked) and hands each layer
        its own for its next forward; returns them (a merging layer's entry is its merged
        weight).  ``check=False``: no read-back (see the
        class documentation); each layer's norm metadata is then that of the last checked
        render."""
        if not check and (self._plan is None or self._key != self._param_key()):
            raise RuntimeError("render(check=False) needs the plan of an earlier checked render() "
                               "with the same parameter tensors and K")
        self._check = bool(check)
        ctx = torch.autocast(device_type="cuda", enabled=False) if self.device.type == "cuda" else _null()
        with ctx:
            params = []
            for ly in self.layers:
                params += [ly.mu_raw, ly.chol_raw, ly.amp]
            deltas = _BatchedFieldFunction.apply(self, *params)
        for ly, d, nrm, kind in zip(self.layers, deltas, self._norms, self._kinds):
            ly.__dict__["_batched_delta"] = (d, nrm, kind)  # a plain attribute (no Module bookkeeping)
        return list(deltas)

    def check(self) -> list[int]:
        """Every layer's pair count of the last forward, from one read-back (synchronises).
        Raises on a device status bit, e.g. a layer whose pairs passed its id capacity during
        unchecked renders."""
        Nat = self._Nat
        status, pairs, self._norms = self._plan.read(clear=True, norms=True)
        bad = [(i, st) for i, st in enumerate(status) if st]
        if bad:
            raise RuntimeError(f"batched fields: device status {bad} (layer, GF_STATUS_* bits; "
                               f"GF_STATUS_CAPACITY = {Nat.GF_STATUS_CAPACITY}: render() with check=True "
                               "grows the id capacities)")
        self._pairs = pairs
        return pairs

    def _run_forward(self) -> list[Tensor]:
        Nat = self._Nat
        if not self._check:
            self._plan.forward()
            return self._deltas
        if self._plan is None or self._key != self._param_key():
            self._build()
        for _ in range(8):
            self._plan.forward()
            status, pairs, self._norms = self._plan.read(clear=True, norms=True)
            over = [i for i, st in enumerate(status) if st & Nat.GF_STATUS_CAPACITY]
            bad = [(i, st) for i, st in enumerate(status) if st & ~Nat.GF_STATUS_CAPACITY]
            if bad:
                raise RuntimeError(f"batched fields: device status {bad} (layer, GF_STATUS_* bits)")
            if not over:
                self._pairs = pairs
                return self._deltas
            for i in over:
                self._caps[i] = max(int(pairs[i] * self.headroom) + 1, self._caps[i] * 2)
            self._build()
        raise RuntimeError("batched fields: id capacities did not settle")

    def _zero_grad(self, i: int) -> Tensor:
        pl = self._plan.plans[i]
        z = self._zero_grads.get(i)
        if z is None or z.numel() != pl.M * pl.N:
            z = torch.zeros(pl.M * pl.N, dtype=torch.float32, device=self.device)
            self._zero_grads[i] = z
        return z

    def _run_backward(self, grads) -> list[Tensor | None]:
        gs = []
        for i, g in enumerate(grads):
            if g is None:
                g = self._zero_grad(i)
            elif g.dtype != torch.float32 or not g.is_contiguous():
                g = g.to(torch.float32).contiguous()
            gs.append(g)
        self._plan.set_grads(gs, check=False)
        self._plan.backward()
        # one copy of every layer's gradients (the plan's buffer is rewritten by the next
        # backward), split into the parameters' shapes
        flat = self._plan.grad_flat[:self._plan.grad_numel].clone()
        return list(torch._utils._unflatten_dense_tensors(flat, self._grad_like))
