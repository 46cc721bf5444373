#!/usr/bin/env python3
"""Benchmark: particle-steps/s of the 2D fixed-NPA rollout at 65,536 particles (C2) on one MI355X.

A "step" is one rollout step of the whole system resident in HBM: hashgrid build,
density pass, fused perception + update MLP + masked Euler update; the C2 decode
(a 512x512 RGBA Gaussian splat of all particles) runs after every 32nd step and is
inside the timed region. Warmup runs on a throwaway copy of the state, so the
timed steps are exactly steps 0..K-1 of C2 from its seeded inputs.

Prints ONE JSON line with the driver's fields plus:
  roofline      - the fused update kernel (the dominant one), its algorithmic fp32
                  work per launch over its mean launch time (HIP events on the
                  library's stream over the timed region), against MI355X fp32 peak;
  roofline_hbm  - the same kernel against the HBM roofline, as BASELINE.json asks;
  cpu_baseline  - the CPU oracle (C restatement of the reference CPU path) timed on
                  a bounded sample of the same workload on this host's cores.

--workload c3 / c4 / c5 time BASELINE's other rollout workloads the same way; --workload render
times the projected 3D render of a device-resident C4 state (particle-views/s, see bench_render);
--workload adjoint times the perception adjoint on C2's particles (see bench_adjoint).
--workload raster times the EWA raster of a C4 state's decoded Gaussians (see bench_raster).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_FP32_TFLOPS = 157.3
# The bit-exact path issues unfused, unpacked fp32 adds and multiplies: one operation per lane per
# cycle, 256 CUs x 64 lanes x 2.4 GHz. The published 157.3 counts fused multiply-adds on packed
# pairs (4 operations per lane per cycle), which a path that must round every product and sum
# separately cannot use.
VALU_CEILING_TOPS = 256 * 64 * 2.4e9 / 1e12
PEAK_HBM_GBS = 8000.0


def cpu_model() -> str:
    try:
        for l in open("/proc/cpuinfo"):
            if l.startswith("model name"):
                return l.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"

# the timed region prices the dominant kernel from event-timed launches on one step in SAMPLE_EVERY
SAMPLE_EVERY = 16
KERNEL_IDS = {"hash_rank": 0, "table_scan": 1, "offsets_scan": 2, "scatter": 3, "density": 4,
              "perceive": 5, "mlp": 7, "split": 8, "update": 12}  # NPA_KERNEL_* in include/npa_abi.h


def kernel_work(model, counts, particles: int):
    """Algorithmic fp32 operations and HBM bytes of one launch of each per-step kernel, counting
    each IEEE add/sub/mul/div/sqrt the reference performs (density-grad-off path; d = spatial
    dims, S = state dims, F/H/O = MLP widths). `counts` holds the step's exact work counters: the
    density pass runs over every particle, the second pass and the update MLP over the targets of
    the update mask (a masked-out particle is copied unchanged, as the reference's GPU step does).
      density  : per candidate slot 5 (delta 2, r^2 3); per accepted pair 5 (poly6 4, sum 1);
                 per particle 1 (volume)
      perceive : per target candidate slot 5; per target pair 4 + 1 + 2S + 7 + d + S(1 + 2d) + 2d^2
                 (poly6, weight, blur, sqrt/t/t^2/magnitude, volume gradient, state gradient,
                 moment; 134 for S=16, d=2); per target 15 + 2Sd^2 + Sd + S(3d + 23)
                 (inverse, correction, scaling, log-norm with log1p ~20)
      mlp      : per target 2(FH + HO) + (3d + 2) + 3d + 3S (MLP, motion, Euler)
    Bytes count each particle's own rows once (neighbour rows are re-reads served by caches):
      density 16 + 4 + 4 per particle; perceive 16 + 4S + 4 + 4 + 4F per target;
      mlp 4F + 4 + 16 + 4S + 16 + 4S per target.
    """
    S, d, H = model.state_dims, model.spatial_dims, model.hidden_dims
    F, O = model.perception_dims(), model.update_dims()
    n = float(particles)
    t = float(counts["targets"])
    per_pair = 4 + 1 + 2 * S + 7 + d + S * (1 + 2 * d) + 2 * d * d
    work = {
        "density": (5.0 * counts["candidates"] + 5.0 * counts["pairs"] + n, n * 24),
        "perceive": (5.0 * counts["target_candidates"] + per_pair * counts["target_pairs"]
                     + t * (15 + 2 * S * d * d + S * d + S * (3 * d + 23)),
                     t * (16 + 4 * S + 8 + 4 * F)),
        "mlp": (t * (2 * (F * H + H * O) + (3 * d + 2) + 3 * d + 3 * S),
                t * (4 * F + 4 + 32 + 8 * S)),
    }
    # the fused kernel (second pass + MLP + Euler): the work of both, feature rows not in HBM
    per = work
    per["update"] = (per["perceive"][0] + per["mlp"][0],
                     t * (16 + 4 * S + 8) + t * (4 + 32 + 8 * S))
    return per


def cpu_baseline(w, budget_s: float):
    """The CPU oracle on this host's cores over a bounded sample of the workload: whole steps from
    the seeded inputs when a step fits the budget, otherwise (C3) one step evaluated at a uniform
    random sample of particles - their density pass and their second pass + MLP + Euler, the
    per-particle work of a full step - scaled to particle-steps/s."""
    import numpy as np
    from oracle import oracle as O

    O.build()
    threads = O.max_threads()
    b, n = w["batch"], w["n"]
    total = n * b
    pos, st = w["positions"], w["states"]
    if total <= 262144:
        t0 = time.perf_counter()
        steps = 0
        while True:
            mask = O.update_mask(b, n, w["update_prob"], steps, w["seed"])
            out = O.step(w["model"], w["weights"], pos, st, b, n, w["grid"], w["dt"], mask)
            pos, st = out.next_positions, out.next_states
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or steps >= 256:
                break
        return {
            "value": total * steps / el, "unit": "particle-steps/sec", "cores": threads,
            "kind": "port", "cpu_model": cpu_model(),
            "sample": (f"first {steps} steps of the same workload from its seeded inputs "
                       f"({total} particles, oracle/libnpa_oracle.so, OpenMP {threads} threads, "
                       f"{el:.1f} s; decode excluded)"),
        }
    mask = O.update_mask(b, n, w["update_prob"], 0, w["seed"])
    rng = np.random.default_rng(0)
    dens = np.zeros(total, np.float32)  # second-pass volumes; the timed work is the same for any
    k, done, el = 256, 0, 0.0
    while el < budget_s and done < total:
        k = min(k, total - done)
        sel = np.sort(rng.choice(total, k, replace=False)).astype(np.uint32)
        t0 = time.perf_counter()
        d = O.density_rows(pos, b, n, w["grid"], sel)
        dens[sel] = d
        O.step_rows(w["model"], w["weights"], pos, st, b, n, w["grid"], w["dt"], mask, dens, sel)
        el += time.perf_counter() - t0
        done += k
        k *= 2
    return {
        "value": done / el, "unit": "particle-steps/sec", "cores": threads, "kind": "port",
        "cpu_model": cpu_model(),
        "sample": (f"step 0 of the same workload evaluated at {done} uniformly sampled particles "
                   f"of {total} (density pass, second pass, MLP and Euler of each; a full "
                   f"oracle step would take {total / (done / el) / 60:.0f} min here), "
                   f"oracle/libnpa_oracle.so, OpenMP {threads} threads, "
                   f"{el:.1f} s"),
    }


RENDER_FLOPS_PER_PIXEL = 29  # per footprint pixel of one particle in one view; see render_work


def render_work(positions, sigmas, views, cfg):
    """Footprint pixels of the projected render (render_loss/image.rs:18-79): for each particle
    and view, the in-bounds part of its (2 ceil(5 sigma) + 1)^2 window. Each footprint pixel costs
    the splat 29 fp32 operations, an exp counted as one: 8 for the weight sum of the first pass
    (dx, dy, dx^2 + dy^2, / 2 sigma^2, exp, sum) and 21 for the accumulation (the same 7, w / denom
    * norm * opacity, 5 multiply-adds into r, g, b, alpha, depth)."""
    import numpy as np

    p = np.asarray(positions, np.float64)[:, :3]
    s = np.clip(np.asarray(sigmas, np.float64), cfg.min_sigma, cfg.max_sigma)
    r = np.maximum(np.ceil(5.0 * s), 1.0)
    size, ws = cfg.image_size, cfg.world_scale
    bases = {0: ((1, 0, 0), (0, 1, 0)), 1: ((1, 0, 0), (0, 0, 1)), 2: ((0, 1, 0), (0, 0, 1)),
             3: (np.array([1, -1, 0]) / np.sqrt(2), np.array([1, 1, 2]) / np.sqrt(6))}
    total = 0.0
    for v in views:
        right, up = (np.asarray(b, np.float64) for b in bases[int(v)])
        px = (p @ right + ws) / (2 * ws) * (size - 1)
        py = (ws - p @ up) / (2 * ws) * (size - 1)
        bx, by = np.floor(px), np.floor(py)
        wx = np.clip(np.minimum(bx + r, size - 1) - np.maximum(bx - r, 0) + 1, 0, None)
        wy = np.clip(np.minimum(by + r, size - 1) - np.maximum(by - r, 0) + 1, 0, None)
        total += float((wx * wy).sum())
    return total


def bench_render(args, torch) -> int:
    """The projected 3D render of a device-resident state: the particle images of
    mesh_multiview_render_loss_from_trace (render_loss.rs:107-141) - render attributes from the
    states, then project_positions + splat_projected for the four views - on C4's 16,384 surface
    particles (S = 16) at the reference's RenderLossConfig defaults (64x64, sigma 2.5 px)."""
    import ctypes as C

    from burn_automata_amd import synthetic as syn
    from burn_automata_amd._lib import lib
    from burn_automata_amd.config import ALL_VIEWS, RenderLossConfig
    from burn_automata_amd.executor import HipAutomataExecutor
    from burn_automata_amd.model import NpaModel

    w = syn.workload("c4", particles=args.particles)
    cfg = RenderLossConfig(image_size=args.image_size or 64)
    ex = HipAutomataExecutor()
    ctx = ex.ctx
    n = w["n"]
    state = ex.create_state(NpaModel(w["model"], w["weights"]), torch.from_numpy(w["positions"]).cuda(),
                            torch.from_numpy(w["states"]).cuda(), 1, n, w["grid"], w["dt"],
                            w["update_prob"], w["seed"])
    for _ in range(args.warmup):
        ex.render_views(state, cfg)
    torch.cuda.synchronize()
    L = lib()
    kid = 10  # NPA_KERNEL_RENDER: the render pipeline after the attributes kernel
    ctx.check(L.npa_profile_reset(ctx.handle))
    ctx.check(L.npa_profile_enable(ctx.handle, 1 << kid))
    t0 = time.perf_counter()
    for _ in range(args.steps):
        img = ex.render_views(state, cfg)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tot, cnt = C.c_double(), C.c_uint64()
    ctx.check(L.npa_profile_read(ctx.handle, kid, C.byref(tot), C.byref(cnt)))
    ctx.check(L.npa_profile_enable(ctx.handle, 0))
    pipe_ms = tot.value / max(cnt.value, 1)
    finite = bool(torch.isfinite(img).all().item())
    state.close()
    views = len(ALL_VIEWS)
    value = n * views * args.steps / elapsed
    pixels = render_work(w["positions"], [cfg.sigma] * n, ALL_VIEWS, cfg)
    flops = pixels * RENDER_FLOPS_PER_PIXEL
    achieved = flops / (pipe_ms * 1e-3) / 1e12
    line = {
        "metric": "particle-views/sec, projected 3D render (render-loss particle images)",
        "value": value, "unit": "particle-views/sec", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1000.0 * elapsed / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (C4 seeded surface particles and states)",
        "config": {"workload": (f"render: C4 state ({n} particles, S={w['model'].state_dims}), "
                                f"{views} views (Xy, Xz, Yz, Iso), {cfg.image_size}x{cfg.image_size} "
                                f"RGBA+depth, sigma {cfg.sigma} px, FixedScale, world_scale "
                                f"{cfg.world_scale}"),
                   "particles": n, "views": views, "image_size": cfg.image_size,
                   "footprint_pixels": pixels, "images_finite": finite},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_FP32_TFLOPS, "traffic": None,
                     "kernel": "render pipeline (prep + scans + key sort + tiles)",
                     "engine": "fp32 VALU; exp counted as one operation",
                     "mean_launch_ms": pipe_ms, "flops_per_launch": flops,
                     "timing": "HIP events around the render pipeline of every timed call, on the "
                               "library's stream"},
    }
    if not args.no_cpu_baseline:
        from oracle import oracle as O

        O.build()
        st = w["states"]
        t0 = time.perf_counter()
        reps = 0
        while True:
            col, op, sg, _ = O.render_attributes(st, w["model"].state_dims, cfg)
            O.render_views(w["positions"], col, op, sg, ALL_VIEWS, cfg)
            reps += 1
            el = time.perf_counter() - t0
            if el >= min(args.cpu_seconds, 20.0) or reps >= 64:
                break
        line["cpu_baseline"] = {
            "value": n * views * reps / el, "unit": "particle-views/sec", "cores": 1, "kind": "port",
            "sample": (f"{reps} renders of the same state and views (oracle/libnpa_oracle.so "
                       f"render_attributes + project_positions + splat_projected, one thread, "
                       f"{el:.1f} s)")}
    print(json.dumps(line), flush=True)
    return 0


def adjoint_work(S: int, d: int, hybrid: bool, state_grad: bool, density_grad: bool, pairs: float,
                 particles: float) -> float:
    """fp32 operations of perceive_adjoint_with_options (adjoint.rs), each add/sub/mul/div/sqrt
    counted once, per ordered accepted pair (self pairs included; they cost the same to visit):
      density pass           10                 (delta, r^2, poly6, sum)
      blurred state          14 + 4S + 5d       (poly6 and its delta adjoint, weight and
                                                 state terms per channel, volume adjoint)
      gradient, first walk   8 + d + S(1 + 2d) + [hybrid] 2d^2
      gradient, second walk  15 + 2d + S(14 + 14d) + [hybrid] 4d^2 + 12d + 13
      density gradient       2 x (10 + 9d)      (its forward sum and the delta adjoint)
      density kernel         4 + 5d
    plus per particle S(6d^2 + 5d + 32) + 120 (moment correction, log-norm adjoint with its
    log1p, inverse and inverse adjoint)."""
    per_pair = 10 + 14 + 4 * S + 5 * d + 4 + 5 * d
    if state_grad:
        per_pair += 8 + d + S * (1 + 2 * d) + (2 * d * d if hybrid else 0)
        per_pair += 15 + 2 * d + S * (14 + 14 * d) + ((4 * d * d + 12 * d + 13) if hybrid else 0)
    if density_grad:
        per_pair += 2 * (10 + 9 * d)
    per_particle = S * (6 * d * d + 5 * d + 32) + 120
    return pairs * per_pair + particles * per_particle


RASTER_FLOPS_PER_PAIR = 25


def bench_raster(args, torch) -> int:
    """The frame the viewer draws from a device-resident state: decode_gaussians_3d of C4's
    16,384 surface particles (FixedScale, colours as RGB) and the EWA raster of the Gaussians
    (npa_state_raster_gaussians_3d) at 1024x1024, the camera framing the surface. Each (pixel,
    Gaussian) evaluation before the pixel's stop costs the compositing loop 25 fp32 operations, an
    exp counted as one (offsets 2, power 8, exp, opacity and clamp 2, floor test, 1 - alpha, T
    product, cut test, colour 9); the count comes from the oracle's raster of the same frame in the
    cpu_baseline leg (null without it)."""
    import ctypes as C

    import numpy as np

    from burn_automata_amd import synthetic as syn
    from burn_automata_amd._lib import lib
    from burn_automata_amd.config import GaussianDecodeConfig, RasterCamera, RasterColor
    from burn_automata_amd.executor import HipAutomataExecutor
    from burn_automata_amd.model import NpaModel

    size = args.image_size or 1024
    w = syn.workload("c4", particles=args.particles)
    ex = HipAutomataExecutor()
    ctx = ex.ctx
    n = w["n"]
    state = ex.create_state(NpaModel(w["model"], w["weights"]), torch.from_numpy(w["positions"]).cuda(),
                            torch.from_numpy(w["states"]).cuda(), 1, n, w["grid"], w["dt"],
                            w["update_prob"], w["seed"])
    dcfg = GaussianDecodeConfig()
    p = w["positions"][:, :3].astype(np.float64)
    centre = p.mean(axis=0)
    ext = float(np.abs(p - centre).max())
    cam = RasterCamera.look_at(tuple(centre + np.array([0.6, 0.9, 2.4]) * ext), tuple(centre), width=size,
                               height=size, color_mode=RasterColor.Rgb)
    for _ in range(args.warmup):
        ex.raster_gaussians_3d(state, dcfg, cam)
    torch.cuda.synchronize()
    L = lib()
    kid = 11  # NPA_KERNEL_RASTER: the raster pipeline after the decode kernel
    ctx.check(L.npa_profile_reset(ctx.handle))
    ctx.check(L.npa_profile_enable(ctx.handle, 1 << kid))
    t0 = time.perf_counter()
    for _ in range(args.steps):
        img = ex.raster_gaussians_3d(state, dcfg, cam)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tot, cnt = C.c_double(), C.c_uint64()
    ctx.check(L.npa_profile_read(ctx.handle, kid, C.byref(tot), C.byref(cnt)))
    ctx.check(L.npa_profile_enable(ctx.handle, 0))
    pipe_ms = tot.value / max(cnt.value, 1)
    coverage = float((img[..., 3] > 0.01).float().mean().item())
    dec = {k: v.cpu().numpy() for k, v in ex.decode_gaussians_3d(state, dcfg).items()}
    state.close()
    line = {
        "metric": "Gaussian-frames/sec, EWA oriented-Gaussian raster of a device-resident state",
        "value": n * args.steps / elapsed, "unit": "Gaussian-frames/sec", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1000.0 * elapsed / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (C4 seeded surface particles and states)",
        "config": {"workload": (f"raster: C4 state ({n} particles, S={w['model'].state_dims}) decoded "
                                f"(GaussianSh0FixedScale) and drawn at {size}x{size}, 16x16 tiles, "
                                f"front-to-back, camera framing the surface"),
                   "particles": n, "image_size": size, "coverage": coverage},
        "roofline": {"bound": "mfma", "achieved": None, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                     "frac": None, "traffic": None,
                     "kernel": "raster pipeline (prep + depth sort + scans + emit + tile sort + tiles)",
                     "engine": "fp32 VALU; exp counted as one operation",
                     "mean_launch_ms": pipe_ms,
                     "timing": "HIP events around the raster pipeline of every timed call, on the "
                               "library's stream"},
    }
    if not args.no_cpu_baseline:
        from oracle import oracle as O

        O.build()
        t0 = time.perf_counter()
        reps = 0
        while True:
            _, pairs = O.raster_gaussians_3d(dec["position_visibility"], dec["spherical_harmonic"],
                                             dec["rotation"], dec["scale_opacity"], cam, return_evaluated=True)
            reps += 1
            el = time.perf_counter() - t0
            if el >= min(args.cpu_seconds, 20.0) or reps >= 64:
                break
        threads = O.max_threads()
        flops = pairs * RASTER_FLOPS_PER_PAIR
        achieved = flops / (pipe_ms * 1e-3) / 1e12
        line["roofline"].update({"achieved": achieved, "frac": achieved / PEAK_FP32_TFLOPS,
                                 "flops_per_launch": flops, "evaluated_pairs": pairs})
        line["cpu_baseline"] = {
            "value": n * reps / el, "unit": "Gaussian-frames/sec", "cores": threads, "kind": "port",
            "sample": (f"{reps} rasters of the same decoded frame (oracle/libnpa_oracle.so "
                       f"oracle_raster_gaussians_3d, {threads} OpenMP threads over tiles, {el:.1f} s)")}
    print(json.dumps(line), flush=True)
    return 0


def bench_adjoint(args, torch) -> int:
    """The perception adjoint (perceive_adjoint_with_options, adjoint.rs:27-136) of C2's 65,536
    particles with the growing-2D model's perception options and a seeded synthetic feature
    adjoint: one call = hashgrid build + the four adjoint passes."""
    import numpy as np

    from burn_automata_amd import kernels as K
    from burn_automata_amd import synthetic as syn
    from burn_automata_amd.runtime import default_context

    w = syn.workload("c2", particles=args.particles)
    m, g = w["model"], w["grid"]
    opts = m.perception_options()
    n, S, d = w["n"], m.state_dims, g.dim
    F = opts.feature_dims(S, d)
    rng = np.random.default_rng(11)
    pos = torch.from_numpy(w["positions"]).cuda()
    st = torch.from_numpy(w["states"]).cuda()
    fa_np = rng.normal(0.0, 0.1, n * F).astype(np.float32)
    fa = torch.from_numpy(fa_np).cuda()
    ctx = default_context()
    for _ in range(args.warmup):
        K.perceive_adjoint_with_options(pos, st, 1, n, S, g, opts, fa, ctx=ctx)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = K.perceive_adjoint_with_options(pos, st, 1, n, S, g, opts, fa, ctx=ctx)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    finite = bool(torch.isfinite(out.state).all().item() and torch.isfinite(out.position).all().item())
    off, _ = K.neighbor_lists(pos, 1, n, g, ctx=ctx)
    pairs = float(off[-1].item())
    ms = 1000.0 * elapsed / args.steps
    flops = adjoint_work(S, d, opts.hybrid_state_gradient, opts.state_grad, opts.density_grad, pairs, n)
    achieved = flops / (ms * 1e-3) / 1e12
    line = {
        "metric": "particle-adjoints/sec, perception adjoint (training backward of the perception)",
        "value": n * args.steps / elapsed, "unit": "particle-adjoints/sec", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (C2 seeded particles and states; feature adjoint N(0, 0.1^2))",
        "config": {"workload": (f"adjoint: C2 particles ({n}), S={S}, F={F}, growing-2D perception "
                                f"options (state gradient, hybrid moment, log-norm), eps={g.eps}"),
                   "particles": n, "pairs": pairs, "outputs_finite": finite},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_FP32_TFLOPS, "traffic": None,
                     "kernel": "whole call (hashgrid build + k_adj_density, k_adj_prep, k_adj_gather, "
                               "k_adj_density_kernel)",
                     "engine": "fp32 VALU", "mean_launch_ms": ms, "flops_per_launch": flops,
                     "timing": "wall clock over the timed calls (synchronised on both sides)"},
    }
    if not args.no_cpu_baseline:
        from oracle import oracle as O

        O.build()
        pos_np, st_np = w["positions"], w["states"]
        t0 = time.perf_counter()
        reps = 0
        while True:
            O.perceive_adjoint_with_options(pos_np, st_np, 1, n, S, g, opts, fa_np)
            reps += 1
            el = time.perf_counter() - t0
            if el >= min(args.cpu_seconds, 20.0) or reps >= 32:
                break
        line["cpu_baseline"] = {
            "value": n * reps / el, "unit": "particle-adjoints/sec", "cores": 1, "kind": "port",
            "sample": (f"{reps} calls of oracle perceive_adjoint_with_options on the same inputs "
                       f"(serial like the reference's loop, one thread, {el:.1f} s)")}
    print(json.dumps(line), flush=True)
    return 0


def copy_calibration(torch, mib: float) -> int:
    n = int(mib * (1 << 20)) // 4
    src = torch.rand(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(8):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"bytes_read": 4 * n, "bytes_written": 4 * n,
                                           "launches": 8}}), flush=True)
    return 0


def recorded_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary (FETCH_SIZE and
    WRITE_SIZE per dispatch, each divided by what the counter reads for a copy of known size)."""
    path = os.path.join(ROOT, "profiles", "c2_hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
            return float(parts[2])
    return None


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--workload", default="c2")
    ap.add_argument("--particles", type=int, default=None)
    ap.add_argument("--image-size", type=int, default=None,
                    help="render (default 64) and raster (default 1024) workloads only")
    ap.add_argument("--decode-every", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--mlp-engine", choices=("valu", "mfma", "bf16"), default="valu",
                    help="update MLP on the vector ALUs in the reference's order (bit-exact, default), "
                         "on the fp32 matrix cores, or with layer 1 on the bf16 matrix cores (bf16x3 "
                         "features, bf16 weights; 2D fused kernel) - both single-step tolerance")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-alt-engine", action="store_true",
                    help="skip the matrix-core engine's run beside the headline")
    ap.add_argument("--no-profile", action="store_true",
                    help="skip the HIP-event bracketing of the per-step kernels")
    ap.add_argument("--skip-replay", action="store_true",
                    help="skip the untimed replay that counts candidates and pairs (profiling runs)")
    ap.add_argument("--copy-calibration", type=float, default=None, metavar="MIB",
                    help="only copy a MIB-sized float32 buffer 8 times (the reference kernel whose "
                         "FETCH_SIZE / WRITE_SIZE counters scale the HBM traffic figures)")
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}, WORLD_SIZE={world}): "
              "this build has no multi-GPU path; the sharding design is described in DESIGN.md",
              file=sys.stderr)
        return 2

    import torch

    if args.copy_calibration is not None:
        return copy_calibration(torch, args.copy_calibration)
    if args.workload == "render":
        return bench_render(args, torch)
    if args.workload == "adjoint":
        return bench_adjoint(args, torch)
    if args.workload == "raster":
        return bench_raster(args, torch)

    from burn_automata_amd import kernels as K
    from burn_automata_amd import synthetic as syn
    from burn_automata_amd._lib import lib
    from burn_automata_amd.executor import HipAutomataExecutor
    from burn_automata_amd.model import NpaModel

    w = syn.workload(args.workload, particles=args.particles)
    decode_every = args.decode_every if args.decode_every is not None else w.get("decode_every", 0)
    decode_steps = set() if args.decode_every is not None else set(w.get("decode_steps", ()))
    splat = w.get("splat")
    camera = w.get("camera")  # C4: the EWA raster of the oriented decode
    has_decode = splat is not None or camera is not None
    model = NpaModel(w["model"], w["weights"])
    ex = HipAutomataExecutor()
    ctx = ex.ctx
    B, N = w["batch"], w["n"]
    pos = torch.from_numpy(w["positions"]).cuda()
    st = torch.from_numpy(w["states"]).cuda()

    def due(k):  # decode after step k (1-based count of steps taken)
        return has_decode and ((decode_every and k % decode_every == 0) or k in decode_steps)

    def decode(state):
        if "tiles_x" in w:  # C5: every system in its own window
            ex.splat_2d_tiled(state, splat, w["tiles_x"])
        elif camera is not None:  # C4: oriented Gaussian decode and its EWA raster, one call
            ex.raster_gaussians_3d(state, w["decode"], camera)
        else:
            ex.splat_2d(state, splat)

    from burn_automata_amd import _abi
    engine = {"valu": _abi.MLP_VALU, "mfma": _abi.MLP_MFMA, "bf16": _abi.MLP_MFMA_BF16}[args.mlp_engine]
    L = lib()

    def new_state():
        st_ = ex.create_state(model, pos, st, B, N, w["grid"], w["dt"], w["update_prob"], w["seed"])
        st_.set_mlp_engine(engine)
        return st_

    def run(state, steps, sample=None):
        # sample = (mask, period): the library times the kernels in `mask` with HIP events on the
        # steps k with k % period == period // 2 only; every other step runs without events
        done = 0
        while done < steps:
            k0 = state.step_index()
            sampled = sample is not None and k0 % sample[1] == sample[1] // 2
            chunk = 1
            while (not sampled and done + chunk < steps and not due(k0 + chunk)
                   and not (sample is not None and (k0 + chunk) % sample[1] == sample[1] // 2)):
                chunk += 1
            if sampled:
                ctx.check(L.npa_profile_enable(ctx.handle, sample[0]))
            ex.step_state_many(state, chunk)
            if sampled:
                ctx.check(L.npa_profile_enable(ctx.handle, 0))
            done += chunk
            if due(state.step_index()):
                decode(state)

    # warmup on a throwaway state; the decode runs once too, so that its first-call costs (code
    # object loading of the library's sort kernels) stay out of the timed region
    if args.warmup > 0:
        ws = new_state()
        run(ws, args.warmup)
        if has_decode:
            decode(ws)
        torch.cuda.synchronize()
        ws.close()

    profile = not args.no_profile
    import ctypes as C

    def read_profile():
        out = {}
        for name, kid in KERNEL_IDS.items():
            tot = C.c_double()
            cnt = C.c_uint64()
            ctx.check(L.npa_profile_read(ctx.handle, kid, C.byref(tot), C.byref(cnt)))
            if cnt.value:
                out[name] = tot.value / cnt.value
        ctx.check(L.npa_profile_enable(ctx.handle, 0))
        ctx.check(L.npa_profile_reset(ctx.handle))
        return out

    # Per-kernel means from an untimed pass of the same steps with HIP events around every step
    # kernel (the events cost a few microseconds each, so the timed region brackets only the
    # dominant kernel, whose live mean prices the roofline).
    kernel_ms = {}
    dominant = None
    if profile:
        ps = new_state()
        ctx.check(L.npa_profile_reset(ctx.handle))
        mask = 0
        for kid in KERNEL_IDS.values():
            mask |= 1 << kid
        ctx.check(L.npa_profile_enable(ctx.handle, mask))
        run(ps, args.steps)
        kernel_ms = read_profile()
        ps.close()
        priced = [k for k in ("density", "perceive", "mlp", "update") if k in kernel_ms]
        dominant = max(priced, key=lambda k: kernel_ms[k]) if priced else None

    state = new_state()
    sample = None
    if dominant is not None:
        # the dominant kernel's live mean: events on every SAMPLE_EVERY-th step of the timed region
        # (an event-timed launch costs ~11 us of queue gaps around it, so timing every launch
        # would add 6 % to the C2 step it measures)
        ctx.check(L.npa_profile_reset(ctx.handle))
        sample = (1 << KERNEL_IDS[dominant], min(SAMPLE_EVERY, max(1, args.steps)))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(state, args.steps, sample)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    elapsed = t1 - t0
    live_n = 0
    if dominant is not None:
        cnt_ = C.c_uint64()
        ctx.check(L.npa_profile_read(ctx.handle, KERNEL_IDS[dominant], None, C.byref(cnt_)))
        live_n = cnt_.value
    live_ms = read_profile().get(dominant) if dominant is not None else None
    _, final_states, _ = ex.read_state(state)
    finite = bool(torch.isfinite(final_states).all().item())
    # The workload's decodes per step (C2/C4: one every decode_every steps; C5: the listed steps
    # of its 256): a run shorter than the decode period still pays its share. One decode of the
    # final state is timed here and the decodes the timed steps owe beyond the ones they ran are
    # added to the elapsed time at that cost.
    decode_rate = 0.0
    if has_decode:
        decode_rate = (1.0 / decode_every) if decode_every else len(decode_steps) / float(w.get("steps", 256))
    decodes_run = sum(1 for k in range(1, args.steps + 1) if due(k))
    decode_ms = None
    owed = max(0.0, args.steps * decode_rate - decodes_run)
    if has_decode:
        decode(state)
        torch.cuda.synchronize()
        td0 = time.perf_counter()
        decode(state)
        torch.cuda.synchronize()
        decode_ms = 1000.0 * (time.perf_counter() - td0)
    state.close()
    elapsed_steps = elapsed
    elapsed = elapsed_steps + owed * (decode_ms or 0.0) * 1e-3

    # The same steps on the matrix-core MLP engine, reported beside the headline (which stays on
    # the bit-exact engine): that engine meets the single-step gate but not the 64-step one.
    alt = None
    if args.mlp_engine == "valu" and not args.no_alt_engine:
        engine_saved = engine
        engine = _abi.MLP_MFMA
        aw = new_state()
        run(aw, min(args.warmup, 4) or 1)
        aw.close()
        astate = new_state()
        torch.cuda.synchronize()
        ta0 = time.perf_counter()
        run(astate, args.steps)
        torch.cuda.synchronize()
        alt_elapsed = time.perf_counter() - ta0 + owed * (decode_ms or 0.0) * 1e-3
        astate.close()
        engine = engine_saved
        alt = {"mlp_engine": "mfma", "value": B * N * args.steps / alt_elapsed,
               "ms_per_step": 1000.0 * alt_elapsed / args.steps,
               "gates": "single step within 1e-5 of the reference (tests/test_gpu_mfma.py); not the "
                        "64-step 1e-3 gate: the rollout is chaotic and the reference itself, started "
                        "one ulp away, drifts as far (same test file)"}

    # exact work counts of the timed trajectory (untimed replay of the same steps)
    keys = ("candidates", "pairs", "targets", "target_candidates", "target_pairs")
    sums = dict.fromkeys(keys, 0)
    if not args.skip_replay:
        rs = new_state()
        for _ in range(args.steps):
            c = ex.work_counts(rs)
            for k in keys:
                sums[k] += c[k]
            ex.step_state(rs)
        rs.close()
    mean = {k: v / max(args.steps, 1) for k, v in sums.items()}

    total = B * N
    value = total * args.steps / elapsed
    line = {
        "metric": "particle-steps/sec, 2D NPA rollout @65,536 particles; % of HBM roofline",
        "value": value,
        "unit": "particle-steps/sec",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1000.0 * elapsed / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded counter-based generator; random-init weights U(-0.1, 0.1))",
        "config": {
            "workload": (f"{args.workload.upper()}: {w['grid'].dim}D fixed NPA rollout, {total} "
                         f"particles (batch {B} x {N}), S={w['model'].state_dims}, "
                         f"F={w['model'].perception_dims()}, H={w['model'].hidden_dims}, "
                         f"O={w['model'].update_dims()}, eps={w['grid'].eps}, Particle hashgrid "
                         + "x".join(str(v) for v in w['grid'].grid_size[:w['grid'].dim])
                         + ", update mask "
                         f"p={w['update_prob']}"
                         + (f", {splat.image_size}x{splat.image_size} RGBA splat every "
                            f"{decode_every} steps" if decode_every and splat else "")
                         + (f", oriented Gaussian decode drawn by the EWA raster at "
                            f"{camera.width}x{camera.height} every {decode_every} steps"
                            if decode_every and camera is not None else "")
                         + (f", {w['tiles_x'] * splat.image_size}x{w['tiles_x'] * splat.image_size}"
                            f" tiled splat after steps {sorted(decode_steps)}"
                            if decode_steps and splat else "")),
            "particles": total,
            "mlp_engine": args.mlp_engine,
            "steps_timed": args.steps,
            "decode_every": decode_every,
            "mean_candidates_per_step": mean["candidates"],
            "mean_pairs_per_step": mean["pairs"],
            "mean_targets_per_step": mean["targets"],
            "final_state_finite": finite,
        },
        "decode": {"ms_per_decode": decode_ms, "decodes_per_step": decode_rate,
                   "decodes_in_timed_steps": decodes_run, "decodes_owed": owed,
                   "steps_wall_ms": 1000.0 * elapsed_steps,
                   "note": "value and ms_per_step include the owed decodes at ms_per_decode each"},
    }
    if alt is not None:
        line["alt_engine"] = alt
    if kernel_ms:
        line["kernel_mean_launch_ms"] = kernel_ms  # untimed instrumented pass of the same steps
    if kernel_ms and not args.skip_replay:
        work = kernel_work(w["model"], mean, total)
        per_kernel = {}
        for name, ms in kernel_ms.items():
            if name not in work:
                continue
            if name == dominant and live_ms:
                ms = live_ms  # measured in the timed region
            fl, by = work[name]
            per_kernel[name] = {"mean_launch_ms": ms, "tflops": fl / (ms * 1e-3) / 1e12,
                                "gbs": by / (ms * 1e-3) / 1e9, "flops_per_launch": fl,
                                "bytes_per_launch": by}
        k = per_kernel[dominant]
        # the matrix-core engine runs both MLP layers on MFMA, in the separate MLP kernel and in the
        # fused update kernel alike; the bit-exact engine takes only layer 1's products from MFMA
        # (one rounding each, as v_mul_f32) and adds everything on the VALU in the reference's order
        on_mfma = args.mlp_engine in ("mfma", "bf16") and dominant in ("mlp", "update")
        if on_mfma and args.mlp_engine == "bf16":
            engine_note = ("layer 1 on the bf16 matrix cores (v_mfma_f32_4x4x4bf16_1k, bf16x3 features, "
                           "bf16 weights), layer 2 on the fp32 matrix cores, neighbour walk and sums on the "
                           "VALU; peak = the published MI355X fp32 peak (the MLP's flops are counted as fp32)")
        elif on_mfma:
            engine_note = ("fp32 matrix cores for both MLP layers (v_mfma_f32_4x4x1f32), neighbour walk "
                           "and sums on the VALU; peak = the published MI355X fp32 peak")
        elif dominant == "update":
            engine_note = ("layer-1 products on the fp32 matrix cores (v_mfma_f32_4x4x1f32 with a -0.0 "
                           "accumulator: each product rounded once, as v_mul_f32), every sum and the "
                           "neighbour walk on the VALU, unfused, in the reference's order (bit-exact "
                           "path); peak = the published MI355X fp32 peak")
        else:
            engine_note = ("fp32 VALU, unfused mul/add in the reference's order (bit-exact path); "
                           "peak = the published MI355X fp32 vector peak")
        line["roofline"] = {
            "bound": "mfma" if on_mfma else "valu", "achieved": k["tflops"], "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s", "frac": k["tflops"] / PEAK_FP32_TFLOPS,
            "attainable_peak": VALU_CEILING_TOPS,
            "frac_attainable": k["tflops"] / VALU_CEILING_TOPS,
            "attainable_note": ("frac_attainable is against unfused, unpacked fp32 VALU issue (256 CUs "
                                "x 64 lanes x 2.4 GHz = 39.3 T op/s): the ceiling of a path that rounds "
                                "every sum as the reference does on the vector ALUs, which is where "
                                "this kernel's sums run whichever engine supplies the products"),
            # the committed counter summary covers the C2 workload only
            "traffic": recorded_traffic(dominant) if args.workload == "c2" and args.particles is None else None,
            "traffic_source": ("profiles/c2_hbm_traffic.txt (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                               "copy-kernel scaled)" if args.workload == "c2" and args.particles is None
                               else "not measured for this workload"), "kernel": dominant,
            "engine": engine_note,
            "mean_launch_ms": k["mean_launch_ms"], "flops_per_launch": k["flops_per_launch"],
            "timing": (f"HIP events around the launches of this kernel on every "
                       f"{min(SAMPLE_EVERY, max(1, args.steps))}th step of the timed region ({live_n} "
                       f"launches), on the library's stream"),
        }
        line["roofline_hbm"] = {
            "bound": "hbm", "achieved": k["gbs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": k["gbs"] / PEAK_HBM_GBS, "kernel": dominant, "bytes_per_launch": k["bytes_per_launch"],
        }
        line["kernels"] = per_kernel
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
