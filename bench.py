#!/usr/bin/env python3
"""Benchmark: Gaussian-field delta-W elements/s for forward + backward on one MI355X.

A step is one forward (binning + render) and one backward (gradient reduction + chain rule),
with inputs resident in HBM, issued through the sync-free C ABI path and replayed from a HIP
graph.  Workloads:
  cfg3 (default, the headline)  one 1280x1280 fp32 delta-W from K=1024 Gaussians
                                (guass_amd.ops.FieldPlan: three forward launches and the
                                one-launch backward_direct, which applies the chain rule per
                                tile; fields it does not take run reduction + finish)
  cfg4                          all 128 attention linears of an SD1.5-shaped UNet, K=1024 each,
                                as one batch (guass_amd.ops.FieldBatchPlan: five launches per
                                step for all layers)
  cfg1, cfg2, cfg5, cfg5c, cfg5s  single fields as cfg3 (cfg5s: cfg5's stress variant, Student-t
                                log-scale scale 1.0)
  delta-apply                   the layer's composition with delta-W over the cfg4 shapes (x of
                                --tokens rows, fp32, forward + backward into delta-W): the
                                reference's row-chunked composition against one merged GEMM
  cfg4-model                    the cfg4 layers as GaussianLinear modules: one training step
                                (delta-W, every layer's forward on --model-tokens rows, autograd
                                backward) with GaussianFieldBatch.render() (one batched launch
                                per phase, one host read-back) against every layer rendering
                                its own through the drop-in gaussian_field_train (eager, both)
All with 16x16 tiles (--tile 32: the reference's training configs' 32x32), 3 sigma, clamp 80.

Prints one JSON line (metric contract of the driver) with two extra objects:
  roofline      the dominant kernel's achieved throughput against MI355X peak; its duration is
                measured live with HIP events on the launch stream around a graph of repeated
                launches of that kernel (replay time / launch count);
  cpu_baseline  the CPU oracle (a from-scratch port of the reference's torch CPU path) timed on
                this host on the same inputs (for cfg4, on a stated subset of the layers);
  fused         (single fields the one-pass kernel takes) the same field through gf_fwd_bwd_fused,
                dL/d(delta) given before the forward: step time, and the one-pass kernel's
                roofline (56 flops per evaluation: the forward's 15 and the backward's 41);
  dropin        (single fields) wall time per call of the path the reference layer calls: the
                drop-in extension's forward + backward and gaussian_field_train + autograd
                backward, each with its host synchronisations, beside torch's own autograd cost
                for a custom Function that does no work.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ΔW elements/sec fwd+bwd at 1280×1280,K=1024; % HBM/VALU roofline"
HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
VALU_FP32_PEAK = 157.3e12  # flop/s, MI355X fp32 vector (packed)
FWD_FLOPS_PER_EVAL = 15    # per (pixel, Gaussian) evaluation, reference forward.cu:346-361
BWD_FLOPS_PER_EVAL = 41    # reference backward.cu:313-351


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    # Default: 5000 graph-replayed steps (about 0.1 s at cfg3, 2.7 s at cfg4): the timed region's
    # fixed start-up cost, about 1.2 ms between the clock's start and the first step's kernel on
    # some boxes (outside the HIP events, inside the wall clock), is 0.24 us a step there
    # instead of 2.4 at 500.  The model-step and delta-apply modes default to 500.
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="cfg3",
                    choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "cfg5c", "cfg5s", "cfg4-model", "delta-apply"])
    ap.add_argument("--tokens", type=int, default=4096, help="delta-apply: rows of x per layer")
    ap.add_argument("--model-tokens", type=int, default=64, help="cfg4-model: rows of x per layer")
    ap.add_argument("--delta-apply", default="merged", choices=["merged", "row_chunk"],
                    help="cfg4-model: how each layer composes its base weight with delta-W")
    ap.add_argument("--skip-per-layer", action="store_true",
                    help="cfg4-model: time the batched step only (no per-layer comparison)")
    ap.add_argument("--tile", type=int, default=16, choices=[16, 32],
                    help="square tile size (the headline metric is quoted on 16x16 tiles)")
    ap.add_argument("--layers", type=int, default=None, help="cfg4: first N of the 128 layers")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of graph replay")
    ap.add_argument("--graph-steps", type=int, default=100,
                    help="steps captured per HIP graph (replay overhead is paid once per graph)")
    ap.add_argument("--kernel-reps", type=int, default=20, help="launches per per-kernel timing graph")
    ap.add_argument("--kernel-replays", type=int, default=25, help="timed replays per kernel graph")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--dropin-calls", type=int, default=200,
                    help="single fields: timed calls of the drop-in path the reference layer takes "
                         "(0: skip); the median goes to the line's `dropin` object")
    ap.add_argument("--dropin-only", action="store_true",
                    help="run only the drop-in calls (e.g. under rocprofv3 --hip-trace) and print them")
    ap.add_argument("--dropin-leg", default="all", choices=["all", "ext", "train", "floor"],
                    help="--dropin-only: which of the drop-in timings to run")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run one device-to-device copy of this many MiB (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    ap.add_argument("--traffic-file", default=None,
                    help="per-kernel HBM bytes per launch measured with rocprofv3 --pmc "
                         "(default: profiles/<config>_hbm_traffic.json)")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 500 if args.config in ("cfg4-model", "delta-apply") else 5000
    if args.traffic_file is None:
        args.traffic_file = str(ROOT / "profiles" / f"{args.config}_hbm_traffic.json")
    return args


def algorithmic_counts(tile_ptr, M: int, N: int, K: int, tile_out: int, tile_in: int) -> dict:
    import torch

    R = (M + tile_out - 1) // tile_out
    C = (N + tile_in - 1) // tile_in
    counts = (tile_ptr[1:] - tile_ptr[:-1]).to(torch.float64).reshape(R, C).cpu()
    rows = torch.full((R,), float(tile_out), dtype=torch.float64)
    rows[-1] = M - (R - 1) * tile_out
    cols = torch.full((C,), float(tile_in), dtype=torch.float64)
    cols[-1] = N - (C - 1) * tile_in
    E = float((counts * rows.reshape(-1, 1) * cols.reshape(1, -1)).sum())
    return {
        "elements": float(M * N),
        "pairs": int(tile_ptr[-1].item()),
        "evals": E,
        # per fwd+bwd: write delta + read dL/ddelta (4 B each per element), read 24 B and
        # write 24 B of parameters / gradients per Gaussian
        "bytes_step": 8.0 * M * N + 48.0 * K,
        "bytes_fwd_render": 4.0 * M * N + 24.0 * K,
        "bytes_bwd": 4.0 * M * N + 48.0 * K,
        "flops_fwd": FWD_FLOPS_PER_EVAL * E,
        "flops_bwd": BWD_FLOPS_PER_EVAL * E,
        # the binning state the forward hands to the backward, reported beside the algorithmic
        # bytes rather than in them: tile_ptr [T+1] and gaussian_ids_sorted [P], int64 each
        "bytes_binning_state": 8.0 * (R * C + 1 + int(tile_ptr[-1].item())),
    }


def sum_counts(items: list[dict]) -> dict:
    return {k: sum(c[k] for c in items) for k in items[0]}


def roofline(bytes_: float, flops: float, seconds: float) -> dict:
    t_hbm = bytes_ / HBM_PEAK
    t_valu = flops / VALU_FP32_PEAK
    if t_valu >= t_hbm:
        ach = flops / seconds / 1e12
        return {"bound": "valu", "achieved": ach, "peak": VALU_FP32_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": ach / (VALU_FP32_PEAK / 1e12)}
    ach = bytes_ / seconds / 1e9
    return {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": ach / (HBM_PEAK / 1e9)}


def traffic_bytes(path: str, config: str, kernel: str):
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, copy-calibrated) from the
    committed rocprofv3 --pmc measurement, or None if there is none for this workload."""
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    if data.get("config") != config:
        return None
    entry = data.get("kernels", {}).get(kernel)
    return None if entry is None else float(entry["hbm_bytes_per_launch"])


def cgroup_cpu_quota() -> float | None:
    """CPUs the cgroup v2 quota allows (cpu.max "quota period"), or None when unlimited."""
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
    except (OSError, ValueError):
        return None
    return None if quota == "max" else float(quota) / float(period)


def cpu_baseline(problems, reps: int, note: str, tile: int = 16) -> dict:
    import torch

    from oracle import field_oracle as fo  # CPU baseline leg only

    affinity = len(os.sched_getaffinity(0))
    quota = cgroup_cpu_quota()
    # every core the process may run on; a cgroup CPU quota below that would only time-slice
    # the extra threads, so it caps the count
    threads = affinity if quota is None else max(1, min(affinity, int(quota)))
    torch.set_num_threads(threads)

    def run():
        for p in problems:
            fo.gaussian_field_fwd_bwd(p.row_coords, p.col_coords, p.mu, p.chol_raw, p.amp, p.grad,
                                      tile, tile, 3.0, False, 80.0)

    run()  # warmup
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    elements = sum(p.out_features * p.in_features for p in problems)
    return {"value": elements / med, "unit": "ΔW elements/s", "cores": torch.get_num_threads(),
            "affinity_cores": affinity, "cgroup_cpu_quota": quota, "kind": "port",
            "sample": f"{note}: fwd+bwd (per-tile loop + autograd), 1 warmup + median of {reps}, "
                      f"{med:.2f} s each"}


def fused_times(plan, q, total, per_run, args, graph_time_us, t_bin_ms) -> dict:
    """The same field through gf_fwd_bwd_fused (dL/d(delta) given up front: the binning, then one
    kernel that renders delta-W and reduces dL/d(delta) with the same exponentials), timed as the
    main step (graph replay of --steps steps); the one-pass kernel's duration is the fused call's
    minus the binning's, both from graphs of repeated launches timed with HIP events on their
    stream."""
    import torch

    dev = plan.device

    def fused():
        plan.fwd_bwd_fused(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, q.grad)

    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for _ in range(3):
            fused()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_run):
            fused()
    for _ in range(max(1, args.warmup // per_run)):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps // per_run):
        graph.replay()
    torch.cuda.synchronize()
    ms = 1e3 * (time.perf_counter() - t0) / args.steps
    if plan.status():
        raise RuntimeError(f"fused: device status {plan.status():#x}")
    t_call_us = graph_time_us([fused])
    t_kernel_s = (t_call_us - t_bin_ms * 1e3) / 1e6
    flops = total["flops_fwd"] + total["flops_bwd"]
    return {"ms_per_step": ms, "value": total["elements"] / (ms / 1e3), "unit": "ΔW elements/s",
            "kernels_us": {"k_bin": t_bin_ms * 1e3, "k_fused16": t_kernel_s * 1e6},
            "roofline": dict(roofline(total["bytes_step"], flops, t_kernel_s), kernel="k_fused16",
                             duration_us=t_kernel_s * 1e6,
                             traffic=traffic_bytes(args.traffic_file, args.config, "k_fused16")),
            "step_roofline": roofline(total["bytes_step"], flops, ms / 1e3),
            "launch": f"hip graph replay, {per_run} steps per graph; binning (2 launches) + k_fused16"}


def dropin_times(q, args, dev) -> dict:
    """Wall time of the path the reference layer calls (gaussian_linear.py:178-190 ->
    runtime.py:273-297): the drop-in extension's forward + backward, and gaussian_field_train's
    forward + autograd backward, each call followed by a device synchronisation; medians over
    --dropin-calls.  Beside them, torch's own cost for a custom autograd Function with the same
    arguments that does no work (its forward returns an empty delta, its backward empty
    gradients): the floor of any implementation behind this interface."""
    import warnings

    import torch

    from guass_amd.cuda_field import ext, runtime

    cfg = (args.tile, args.tile, 3.0, False, 80.0)
    mu, raw, amp = (t.clone().requires_grad_(True) for t in (q.mu, q.chol_raw, q.amp))
    kw = dict(row_coords=q.row_coords, col_coords=q.col_coords, tile_out=args.tile, tile_in=args.tile,
              sigma_multiplier=3.0, normalize=False, clamp_quad=80.0)
    n_el = q.row_coords.numel() * q.col_coords.numel()

    class _Floor(torch.autograd.Function):
        @staticmethod
        def forward(ctx, row_coords, col_coords, mu, chol_raw, amp, *rest):
            ctx.save_for_backward(row_coords, col_coords, mu, chol_raw, amp)
            return torch.empty(n_el, device=mu.device)

        @staticmethod
        def backward(ctx, g):
            _, _, mu, chol_raw, amp = ctx.saved_tensors
            return (None, None, torch.empty_like(mu), torch.empty_like(chol_raw), torch.empty_like(amp)) + (None,) * 5

    def ext_call():
        d, tp, ids, ws = ext.forward_with_workspace(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, *cfg)
        ext.gaussian_field_backward(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, tp, ids, *cfg,
                                    forward_workspace=ws)

    def train_call():
        for t in (mu, raw, amp):
            t.grad = None
        runtime.gaussian_field_train(mu=mu, chol_raw=raw, amp=amp, **kw).backward(q.grad)

    def floor_call():
        for t in (mu, raw, amp):
            t.grad = None
        _Floor.apply(q.row_coords, q.col_coords, mu, raw, amp, *cfg).backward(q.grad)

    def median_us(fn) -> float:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(args.dropin_calls):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        return 1e6 * statistics.median(times)

    legs = {"ext": ("ext_fwd_bwd_us", ext_call), "train": ("train_autograd_fwd_bwd_us", train_call),
            "floor": ("torch_autograd_floor_us", floor_call)}
    leg = getattr(args, "dropin_leg", "all")
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # the training Function's one-time notice
        out = {name: median_us(fn) for key, (name, fn) in legs.items() if leg in ("all", key)}
    out.update({"calls": args.dropin_calls, "host_syncs_per_call": 2,
                "note": "medians of forward + backward + torch.cuda.synchronize() per call; host syncs: the "
                        "forward's pair count (sizes gaussian_ids_sorted, as the reference) and the "
                        "backward's saved-state status word"})
    return out


def model_bench(args) -> int:
    """cfg4-model: one training step of the 128 SD1.5 attention layers as GaussianLinear
    modules: every layer's delta-W (GaussianFieldBatch.render(), or each layer rendering its own
    through gaussian_field_train inside its forward, as the reference does), every layer's
    forward on --model-tokens rows of input, and autograd's backward through them."""
    import torch

    from guass_amd import workloads as wl
    from guass_amd.layers import GaussianAdapterConfig, GaussianFieldBatch, GaussianLinear

    dev = torch.device("cuda:0")
    probs = wl.cfg4(args.seed, layers=args.layers)
    layers = []
    for p in probs:
        cfg = GaussianAdapterConfig(init_num_gaussians=p.k, tile_out=16, tile_in=16, delta_apply=args.delta_apply)
        ly = GaussianLinear(p.in_features, p.out_features, adapter_config=cfg, device=dev)
        with torch.no_grad():
            ly.row_coords.copy_(p.row_coords.to(dev))
            ly.col_coords.copy_(p.col_coords.to(dev))
        ly.load_adapter_state({"mu_raw": torch.atanh(p.mu.clamp(-0.999999, 0.999999)),
                               "chol_raw": p.chol_raw, "amp": p.amp})
        layers.append(ly)
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    xs = [torch.randn(args.model_tokens, p.in_features, device=dev, generator=gen) for p in probs]
    gys = [torch.randn(args.model_tokens, p.out_features, device=dev, generator=gen) for p in probs]
    params = [t for ly in layers for t in (ly.mu_raw, ly.chol_raw, ly.amp)]
    fb = GaussianFieldBatch(layers, k_capacity=2 * max(p.k for p in probs))

    def batched():
        fb.render()  # every layer's delta-W, one read-back; each layer's forward consumes its own
        torch.autograd.backward([ly(x) for ly, x in zip(layers, xs)], gys)

    def batched_unchecked():  # the same step without the read-back (checked once afterwards)
        fb.render(check=False)
        torch.autograd.backward([ly(x) for ly, x in zip(layers, xs)], gys)

    def per_layer():  # the reference's step: each layer renders its delta-W in its forward
        torch.autograd.backward([ly(x) for ly, x in zip(layers, xs)], gys)

    def timed(fn, steps: int, warmup: int) -> float:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            for t in params:
                t.grad = None
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    t_batch = timed(batched, args.steps, args.warmup)
    t_unchecked = timed(batched_unchecked, args.steps, args.warmup)
    fb.check()  # one read-back after the unchecked steps (raises on a status bit)
    # torch's share: the same 128 GEMMs (forward, weight gradient) through autograd on plain
    # fp32 weights, with no field at all -- the floor of any step through the layer API
    plain_w = [ly.weight.detach().clone().requires_grad_(True) for ly in layers]

    def gemms_only():
        for w in plain_w:
            w.grad = None
        torch.autograd.backward([torch.nn.functional.linear(x, w) for w, x in zip(plain_w, xs)], gys)

    t_floor = timed(gemms_only, args.steps, args.warmup)
    if args.skip_per_layer:  # e.g. to trace the batched steps alone
        print(json.dumps({"config": "cfg4-model", "batched_ms_per_step": t_batch * 1e3,
                          "unchecked_ms_per_step": t_unchecked * 1e3,
                          "torch_gemm_autograd_floor_ms_per_step": t_floor * 1e3,
                          "steps": args.steps, "warmup": args.warmup}), flush=True)
        return 0
    t_single = timed(per_layer, max(1, args.steps // 5), max(1, args.warmup // 5))
    densify = densify_costs(fb, layers, batched, params)
    elements = float(sum(p.out_features * p.in_features for p in probs))
    out = {
        "metric": "ΔW elements/sec fwd+bwd of the SD1.5 attention layers through the layer API",
        "value": elements / t_batch, "unit": "ΔW elements/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": t_batch * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded Gaussian fields, BASELINE.json cfg4 distribution)",
        "config": {"workload": f"cfg4 x{len(probs)} GaussianLinear layers: GaussianFieldBatch.render, every "
                               f"layer's forward on {args.model_tokens} rows, autograd backward (eager)",
                   "layers": len(probs), "sum_out_x_in": int(elements), "k_per_layer": 1024,
                   "tokens_per_layer": args.model_tokens, "delta_apply": args.delta_apply},
        "unchecked_ms_per_step": t_unchecked * 1e3,
        "torch_gemm_autograd_floor_ms_per_step": t_floor * 1e3,
        "per_layer_ms_per_step": t_single * 1e3,
        "speedup_vs_per_layer": t_single / t_batch,
        "densify": densify,
    }
    print(json.dumps(out), flush=True)
    return 0


def densify_costs(fb, layers, step, params) -> dict:
    """Cost of a densification event (the reference clones up to max_new_gaussians_per_step = 2
    Gaussians per layer every 50 steps, configs/dreambooth_sd_k*_densify.yaml:55-62): every
    layer's parameters replaced by tensors with two more Gaussians, then the in-place re-plan,
    the first step after it, and a plan built from scratch for comparison."""
    import torch

    from guass_amd.layers import GaussianFieldBatch

    allocs = sum(pl.allocations for pl in fb._plan.plans)
    for ly in layers:
        idx = torch.tensor([0, 1], device=ly.mu_raw.device)
        p = ly.get_gaussian_parameters()
        ly.replace_gaussian_parameters_(mu_raw=torch.cat([p["mu_raw"].detach(), p["mu_raw"].detach()[idx]]),
                                        chol_raw=torch.cat([p["chol_raw"].detach(), p["chol_raw"].detach()[idx]]),
                                        amp=torch.cat([p["amp"].detach(), p["amp"].detach()[idx]]))
    params[:] = [t for ly in layers for t in (ly.mu_raw, ly.chol_raw, ly.amp)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fb._build()
    torch.cuda.synchronize()
    replan = time.perf_counter() - t0
    t0 = time.perf_counter()
    step()
    torch.cuda.synchronize()
    first = time.perf_counter() - t0
    t0 = time.perf_counter()
    fresh = GaussianFieldBatch(layers, k_capacity=fb._kcaps)
    fresh._build()
    torch.cuda.synchronize()
    rebuild = time.perf_counter() - t0
    return {"replan_in_place_ms": replan * 1e3, "first_step_after_ms": first * 1e3,
            "plan_from_scratch_ms": rebuild * 1e3,
            "buffers_reallocated": sum(pl.allocations for pl in fb._plan.plans) - allocs}


def delta_apply_bench(args) -> int:
    """delta-apply: forward + backward (into delta-W and x) of y = x (W + delta-W)^T + b over the
    SD1.5 attention shapes, composed as the reference layer does (base GEMM, output clone,
    delta-W GEMMs in row chunks, gaussian_linear.py:222-253) and as one merged GEMM."""
    import torch
    import torch.nn.functional as F

    from guass_amd import workloads as wl

    dev = torch.device("cuda:0")
    shapes = wl.sd15_attention_shapes()[: args.layers]
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    layers = []
    for _, m, n in shapes:
        W = torch.randn(m, n, device=dev, generator=gen) * 0.02
        b = torch.zeros(m, device=dev)
        dW = (torch.randn(m, n, device=dev, generator=gen) * 1e-3).requires_grad_(True)
        x = torch.randn(args.tokens, n, device=dev, generator=gen).requires_grad_(True)
        layers.append((W, b, dW, x, torch.randn(args.tokens, m, device=dev, generator=gen)))

    def row_chunk(W, b, dW, x):
        chunk = min(W.shape[0], 64)
        out = F.linear(x, W, b).clone()
        for r0 in range(0, W.shape[0], chunk):
            out[..., r0:r0 + chunk].add_(F.linear(x, dW[r0:r0 + chunk, :], None))
        return out

    def merged(W, b, dW, x):
        return F.linear(x, W + dW, b)

    def step(fn):
        for W, b, dW, x, g in layers:
            dW.grad = None
            x.grad = None
            fn(W, b, dW, x).backward(g)

    def timed(fn) -> float:
        for _ in range(max(1, args.warmup // 10)):
            step(fn)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        n = max(1, args.steps // 10)
        for _ in range(n):
            step(fn)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n

    t_chunk, t_merged = timed(row_chunk), timed(merged)
    flops = sum(6.0 * args.tokens * m * n for _, m, n in shapes)  # fwd + two backward GEMMs
    out = {
        "metric": "delta-W composition, forward + backward over the SD1.5 attention shapes",
        "value": flops / t_merged / 1e12, "unit": "TFLOP/s (merged)", "n_gpus": 1,
        "steps": max(1, args.steps // 10), "warmup": max(1, args.warmup // 10),
        "ms_per_step": t_merged * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{len(shapes)} SD1.5 attention linears, x of {args.tokens} rows"},
        "row_chunk_ms_per_step": t_chunk * 1e3, "speedup_vs_row_chunk": t_chunk / t_merged,
    }
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "this build has no multi-GPU path to time.", file=sys.stderr)
        return 2
    if args.config == "cfg4-model":
        return model_bench(args)
    if args.config == "delta-apply":
        return delta_apply_bench(args)

    import torch

    from guass_amd import _native as Nat
    from guass_amd import workloads as wl
    from guass_amd.cuda_field import ext
    from guass_amd.ops import FieldBatchPlan, FieldPlan

    dev = torch.device("cuda:0")
    if args.calibrate_copy_mib > 0:
        n = args.calibrate_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    batched = args.config == "cfg4"
    probs = wl.cfg4(args.seed, layers=args.layers) if batched else [wl.CONFIGS[args.config](args.seed)]
    qs = [p.to(dev) for p in probs]
    if args.dropin_only:
        if batched:
            print("--dropin-only times a single field", file=sys.stderr)
            return 2
        print(json.dumps({"config": args.config, "dropin": dropin_times(qs[0], args, dev)}), flush=True)
        return 0
    # Pair count of every field (one synchronising drop-in forward each), then sync-free plans.
    counts = []
    for p, q in zip(probs, qs):
        _, tp0, _ = ext.gaussian_field_forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp,
                                               args.tile, args.tile, 3.0, False, 80.0)
        counts.append(algorithmic_counts(tp0, p.out_features, p.in_features, p.k, args.tile, args.tile))
    total = sum_counts(counts)

    if batched:
        batch = FieldBatchPlan(qs, dev, capacities=[c["pairs"] for c in counts], tile_out=args.tile,
                               tile_in=args.tile)

        def step():
            batch.forward()
            batch.backward()

        phases = {
            "k_bin": [lambda: batch.forward(Nat.GF_PHASE_BIN)],
            "k_emit+": [lambda: batch.forward(Nat.GF_PHASE_BIN | Nat.GF_PHASE_EMIT)],
            "k_render": [lambda: batch.forward(Nat.GF_PHASE_RENDER)],
            "k_bwd": [lambda: batch.backward(Nat.GF_PHASE_REDUCE)],
            "k_bwd_finish": [lambda: batch.backward(Nat.GF_PHASE_FINISH)],
        }
        status = lambda: max(batch.status())  # noqa: E731
        emits = batch.info.emit_blocks > 0
    else:
        q, P = qs[0], counts[0]["pairs"]
        plan = FieldPlan(probs[0].out_features, probs[0].in_features, probs[0].k, dev, ids_capacity=P,
                         tile_out=args.tile, tile_in=args.tile)

        # The backward in one launch where the field allows it (gf_backward_direct: the chain
        # rule applied per tile, no finish pass); elsewhere the same call runs two.  The widest
        # tile rectangle takes part in the choice as in training (gf_backward_train).
        plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
        _, span = plan.bin_info()
        direct_one = plan.direct_launches(P, span) == 1

        def step():
            plan.forward(q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp)
            plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, q.amp, num_pairs=P,
                                 max_span=span)

        phases = {
            "k_bin": [lambda: plan.bin(q.mu, q.chol_raw, q.amp)],
            "k_emit+": [lambda: plan.bin(q.mu, q.chol_raw, q.amp), lambda: plan.emit(q.mu, q.amp)],
            "k_render": [lambda: plan.render(q.row_coords, q.col_coords)],
        }
        if direct_one:
            phases["k_bwd"] = [lambda: plan.backward_direct(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw,
                                                            q.amp, num_pairs=P, max_span=span)]
        else:
            phases["k_bwd"] = [lambda: plan.backward_reduce(q.grad, q.row_coords, q.col_coords, q.mu, q.chol_raw, P)]
            phases["k_bwd_finish"] = [lambda: plan.backward_finish(q.chol_raw, q.amp)]
        status = plan.status
        emits = probs[0].k > 8192 or args.tile not in (16, 32)  # the emission path (no masks)

    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        for _ in range(3):
            step()
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize()
    graph = None
    per_run = 1
    if not args.no_graph:
        # A graph of `per_run` consecutive steps, per_run dividing --steps so that exactly
        # --steps steps are timed.
        per_run = max(1, min(args.graph_steps, args.steps))
        while args.steps % per_run:
            per_run -= 1
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(per_run):
                step()
    run = graph.replay if graph is not None else step

    for _ in range(max(1, args.warmup // per_run)):
        run()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps // per_run):
        run()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = 1e3 * wall / args.steps
    st = status()
    if st:
        print(f"device status bits {st:#x} after the timed run", file=sys.stderr)
        return 1

    # Per-kernel durations: each kernel captured `--kernel-reps` times back to back in one HIP
    # graph, replayed on a side stream bracketed by HIP events recorded on that same stream; the
    # duration is the replay time over the launch count, which matches what rocprofv3's kernel
    # trace reports for the same launches (back-to-back kernels, no host gaps).  Every kernel is
    # idempotent under repetition except k_emit (its fill counters advance), so k_emit is timed
    # as (k_bin + k_emit) minus k_bin; repeated k_bwd only grows the accumulators, which the
    # trailing k_bwd_finish clears (the direct backward's only grow the gradients the next
    # forward clears).
    def graph_time_us(fns) -> float:
        s = torch.cuda.Stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for _ in range(args.kernel_reps):
                    for fn in fns:
                        fn()
            g.replay()
            times = []
            for _ in range(args.kernel_replays):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(s)
                g.replay()
                e1.record(s)
                e1.synchronize()
                times.append(e0.elapsed_time(e1) * 1e3 / args.kernel_reps)
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize()
        return statistics.median(times)

    if not emits:  # the mask path launches no emission kernel
        phases.pop("k_emit+")
    ph = {name: graph_time_us(fns) for name, fns in phases.items()}
    if emits:
        ph["k_emit"] = ph.pop("k_emit+") - ph["k_bin"]
    ph = {k: ph[k] / 1e3 for k in ("k_bin", "k_emit", "k_render", "k_bwd", "k_bwd_finish") if k in ph}  # ms
    step()  # leave the plan in the state of one clean step
    torch.cuda.synchronize()

    value = total["elements"] / (ms_per_step / 1e3)
    kernel_rooflines = {
        "k_render": roofline(total["bytes_fwd_render"], total["flops_fwd"], ph["k_render"] / 1e3),
        "k_bwd": roofline(total["bytes_bwd"], total["flops_bwd"], ph["k_bwd"] / 1e3),
    }
    dominant = max(kernel_rooflines, key=lambda k: ph[k])
    roof = dict(kernel_rooflines[dominant])
    roof.update({"kernel": dominant, "traffic": traffic_bytes(args.traffic_file, args.config, dominant),
                 "duration_us": ph[dominant] * 1e3})
    step_roof = roofline(total["bytes_step"], total["flops_fwd"] + total["flops_bwd"], ms_per_step / 1e3)
    if batched:
        workload = (f"cfg4 SD1.5 attention linears x{len(probs)} (one batch) fwd+bwd, {args.tile}x{args.tile} "
                    "tiles, 3 sigma, clamp 80")
        shape = {"layers": len(probs), "sum_out_x_in": int(total["elements"]), "k_per_layer": 1024}
    else:
        p = probs[0]
        workload = f"{p.name} fwd+bwd, {args.tile}x{args.tile} tiles, 3 sigma, clamp 80"
        shape = {"out_features": p.out_features, "in_features": p.in_features, "k": p.k}
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "ΔW elements/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Gaussian field, BASELINE.json distribution)",
        "config": {"workload": workload, **shape, "pairs": int(total["pairs"]),
                   "pair_pixel_evals": total["evals"],
                   "binning_state_bytes": int(total["bytes_binning_state"]),
                   "launch": (f"hip graph replay, {per_run} steps per graph" if graph is not None
                              else "eager")},
        "roofline": roof,
        "step_roofline": step_roof,
        "kernels_us": {k: v * 1e3 for k, v in ph.items()},
        "kernel_rooflines": kernel_rooflines,
        "gpu_event_ms_per_step": gpu_ms / args.steps,
    }
    if not batched:
        out["config"]["max_span"] = span
        out["config"]["backward_launches"] = 1 if direct_one else 2
    if not batched and plan.fused_supported(span):
        out["fused"] = fused_times(plan, q, total, per_run, args, graph_time_us, ph["k_bin"])
    if not batched and args.dropin_calls > 0:
        out["dropin"] = dropin_times(qs[0], args, dev)
    if not args.no_cpu_baseline:
        if batched:
            sub = probs[:2]
            note = (f"cfg4 seed {args.seed}, first {len(sub)} of {len(probs)} layers "
                    f"({'+'.join(f'{p.out_features}x{p.in_features}' for p in sub)})")
        else:
            sub = probs
            note = f"{probs[0].name} seed {args.seed}, the full layer"
        out["cpu_baseline"] = cpu_baseline(sub, args.cpu_reps, note, args.tile)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
