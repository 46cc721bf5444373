"""The operator surface of ``burn_automata_kernels`` on the MI355X (HIP) path.

Each function keeps the reference's name, argument meaning and error behaviour
and returns freshly allocated device tensors, as the reference returns owned Vecs:

* ``build_hashgrid``          crates/burn_automata_kernels/src/hashgrid.rs:16-69
* ``perceive`` / ``perceive_with_options``
                              crates/burn_automata_kernels/src/reference/forward.rs:3-143
* ``perceive_adjoint_with_options`` / ``perceive_state_adjoint_with_options``
                              crates/burn_automata_kernels/src/reference/adjoint.rs:3-136
* ``euler_step``              crates/burn_automata_kernels/src/reference/step.rs:4-55
* ``decode_gaussians_3d``     crates/burn_automata_kernels/src/gaussian.rs:53-100
* ``splat_particles_2d``      crates/burn_automata_kernels/src/splat.rs:30-93
* ``render_views``            crates/burn_automata/src/render_loss/projection.rs:11-29 +
                              render_loss/image.rs:18-79 (project_positions + splat_projected)
* ``render_attributes``       crates/burn_automata/src/render_loss/attributes.rs:15-87

Inputs may be CUDA tensors (used in place) or host arrays (uploaded first).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _abi
from ._lib import lib
from .config import (ALL_VIEWS, GaussianDecodeConfig, RasterCamera, HashGridConfig, PerceptionOptions,
                     RenderLossConfig, Splat2dConfig)
from .runtime import default_context, device_f32, ptr


def _torch():
    import torch
    return torch


@dataclass
class HashGridSnapshot:
    """HashGridSnapshot (hashgrid.rs:3-14) with u32 index tables on the device."""

    batch_size: int
    particle_count: int
    cell_count: int
    bin_offsets: object
    permutation: object
    inverse_permutation: object


def _positions(positions, expected: int, ctx):
    pos = device_f32(positions, device=ctx.device).reshape(-1, 4) if _numel(positions) else \
        _torch().zeros((0, 4), dtype=_torch().float32, device=f"cuda:{ctx.device}")
    if pos.shape[0] != expected:
        raise _abi.PositionShape(
            f"positions length {pos.shape[0]} does not match batch_size * particle_count {expected}")
    return pos


def _numel(x) -> int:
    try:
        return int(x.numel())
    except AttributeError:
        return int(np.asarray(x).size)


def _states(states, expected: int, ctx):
    st = device_f32(states, device=ctx.device).reshape(-1) if _numel(states) else \
        _torch().zeros(0, dtype=_torch().float32, device=f"cuda:{ctx.device}")
    if st.numel() != expected:
        raise _abi.StateShape(
            f"state length {st.numel()} does not match batch_size * particle_count * state_dims "
            f"{expected}")
    return st


def build_hashgrid(positions, batch_size: int, particle_count: int, cfg: HashGridConfig,
                   ctx=None) -> HashGridSnapshot:
    ctx = ctx or default_context()
    torch = _torch()
    total = batch_size * particle_count
    pos = _positions(positions, total, ctx)
    cells = cfg.cell_count() if cfg.dim in (2, 3) else 0
    dev = f"cuda:{ctx.device}"
    bo = torch.empty(batch_size * cells + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(total, dtype=torch.int32, device=dev)
    inv = torch.empty(total, dtype=torch.int32, device=dev)
    ctx.check(lib().npa_build_hashgrid(ctx.handle, ptr(pos), batch_size, particle_count,
                                       C.byref(cfg.to_c()), ptr(bo), bo.numel(), ptr(perm),
                                       ptr(inv), total))
    return HashGridSnapshot(batch_size, particle_count, cells, bo, perm, inv)


def neighbor_lists(positions, batch_size: int, particle_count: int, cfg: HashGridConfig, ctx=None):
    """Ordered neighbour lists (CSR) exactly as for_each_neighbor visits them (neighbor.rs:3-44)."""
    ctx = ctx or default_context()
    torch = _torch()
    total = batch_size * particle_count
    pos = _positions(positions, total, ctx)
    dev = f"cuda:{ctx.device}"
    off = torch.empty(total + 1, dtype=torch.int32, device=dev)
    need = C.c_size_t()
    ctx.check(lib().npa_neighbor_lists(ctx.handle, ptr(pos), batch_size, particle_count,
                                       C.byref(cfg.to_c()), ptr(off), None, 0, C.byref(need)))
    idx = torch.empty(max(need.value, 1), dtype=torch.int32, device=dev)
    ctx.check(lib().npa_neighbor_lists(ctx.handle, ptr(pos), batch_size, particle_count,
                                       C.byref(cfg.to_c()), ptr(off), ptr(idx), idx.numel(),
                                       C.byref(need)))
    return off, idx[: need.value]


@dataclass
class PerceptionOutput:
    """PerceptionOutput (crates/burn_automata_kernels/src/reference/types.rs:33-41)."""

    features: object
    density: object
    blurred_state: object
    state_gradient: object
    density_gradient: object
    feature_dims: int


def perceive_with_options(positions, states, batch_size: int, particle_count: int,
                          state_dims: int, cfg: HashGridConfig, options: PerceptionOptions,
                          ctx=None) -> PerceptionOutput:
    ctx = ctx or default_context()
    torch = _torch()
    total = batch_size * particle_count
    pos = _positions(positions, total, ctx)
    st = _states(states, total * state_dims, ctx)
    d = cfg.dim
    F = options.feature_dims(state_dims, d)
    dev = f"cuda:{ctx.device}"
    feats = torch.empty((total, F), dtype=torch.float32, device=dev)
    dens = torch.empty(total, dtype=torch.float32, device=dev)
    blur = torch.empty((total, state_dims), dtype=torch.float32, device=dev)
    sg = torch.empty((total, state_dims * d) if options.state_grad else (0,), dtype=torch.float32,
                     device=dev)
    dg = torch.empty((total, d) if options.density_grad else (0,), dtype=torch.float32,
                     device=dev)
    fd = C.c_uint32()
    ctx.check(lib().npa_perceive(ctx.handle, ptr(pos), ptr(st), batch_size, particle_count,
                                 state_dims, C.byref(cfg.to_c()), C.byref(options.to_c()),
                                 ptr(feats), feats.numel(), ptr(dens), ptr(blur),
                                 ptr(sg) if sg.numel() else None, ptr(dg) if dg.numel() else None,
                                 C.byref(fd)))
    return PerceptionOutput(feats, dens, blur, sg, dg, int(fd.value))


@dataclass
class PerceptionAdjointOutput:
    """PerceptionAdjointOutput (reference/types.rs:43-47): state [T * S], position [T, 4]."""

    state: object
    position: object


def perceive_adjoint_with_options(positions, states, batch_size: int, particle_count: int,
                                  state_dims: int, cfg: HashGridConfig, options: PerceptionOptions,
                                  feature_adjoint, ctx=None) -> PerceptionAdjointOutput:
    """perceive_adjoint_with_options (reference/adjoint.rs:27-136) on the device."""
    ctx = ctx or default_context()
    torch = _torch()
    total = batch_size * particle_count
    pos = _positions(positions, total, ctx)
    st = _states(states, total * state_dims, ctx)
    fa = device_f32(feature_adjoint, device=ctx.device).reshape(-1)
    dev = f"cuda:{ctx.device}"
    sa = torch.empty(total * state_dims, dtype=torch.float32, device=dev)
    pa = torch.empty((total, 4), dtype=torch.float32, device=dev)
    ctx.check(lib().npa_perceive_adjoint(ctx.handle, ptr(pos), ptr(st), batch_size, particle_count,
                                         state_dims, C.byref(cfg.to_c()), C.byref(options.to_c()),
                                         ptr(fa), fa.numel(), ptr(sa), ptr(pa)))
    return PerceptionAdjointOutput(sa, pa)


def perceive_state_adjoint_with_options(positions, states, batch_size: int, particle_count: int,
                                        state_dims: int, cfg: HashGridConfig,
                                        options: PerceptionOptions, feature_adjoint, ctx=None):
    """perceive_state_adjoint_with_options (reference/adjoint.rs:3-25)."""
    return perceive_adjoint_with_options(positions, states, batch_size, particle_count, state_dims,
                                         cfg, options, feature_adjoint, ctx).state


def perceive(positions, states, batch_size, particle_count, state_dims, cfg: HashGridConfig,
             state_grad: bool, density_grad: bool, ctx=None) -> PerceptionOutput:
    """perceive (forward.rs:3-23): PerceptionOptions::new(state_grad, density_grad, cfg.eps)."""
    return perceive_with_options(positions, states, batch_size, particle_count, state_dims, cfg,
                                 PerceptionOptions.new(state_grad, density_grad, cfg.eps), ctx)


def euler_step(positions, states, dx, ds, batch_size: int, particle_count: int, state_dims: int,
               cfg: HashGridConfig, dt: float, update_mask=None, ctx=None):
    ctx = ctx or default_context()
    torch = _torch()
    total = batch_size * particle_count
    pos = _positions(positions, total, ctx)
    st = _states(states, total * state_dims, ctx)
    dxt = device_f32(dx, device=ctx.device).reshape(-1, 4)
    dst = device_f32(ds, device=ctx.device).reshape(-1)
    if dxt.shape[0] != total:
        raise _abi.OutputShape(f"output buffer length {dxt.shape[0]} does not match expected {total}")
    if dst.numel() != st.numel():
        raise _abi.OutputShape(
            f"output buffer length {dst.numel()} does not match expected {st.numel()}")
    m = None if update_mask is None else device_f32(update_mask, device=ctx.device).reshape(-1)
    op = torch.empty_like(pos)
    os_ = torch.empty_like(st)
    ctx.check(lib().npa_euler_step(ctx.handle, ptr(pos), ptr(st), ptr(dxt), ptr(dst), batch_size,
                                   particle_count, state_dims, C.byref(cfg.to_c()), float(dt),
                                   ptr(m), ptr(op), ptr(os_)))
    return op, os_.reshape(total, state_dims)


def update_mask(batch_size: int, particle_count: int, update_prob: float, step_index: int,
                seed: int, ctx=None):
    """The device update mask (gpu_step.wgsl:1019-1056; lane seeds state.rs:1282-1315)."""
    ctx = ctx or default_context()
    torch = _torch()
    m = torch.empty(batch_size * particle_count, dtype=torch.float32, device=f"cuda:{ctx.device}")
    ctx.check(lib().npa_update_mask(ctx.handle, batch_size, particle_count, float(update_prob),
                                    int(step_index) & 0xFFFFFFFF, int(seed) & 0xFFFFFFFFFFFFFFFF,
                                    ptr(m)))
    return m


def decode_gaussians_3d(positions, states, state_dims: int, cfg: GaussianDecodeConfig, ctx=None):
    """Planar Gaussian parameters: position_visibility [n,4], spherical_harmonic [n,K,3],
    rotation [n,4], scale_opacity [n,4]."""
    ctx = ctx or default_context()
    torch = _torch()
    pos = device_f32(positions, device=ctx.device).reshape(-1, 4)
    st = device_f32(states, device=ctx.device).reshape(-1)
    n = pos.shape[0]
    if st.numel() != n * state_dims:
        raise AssertionError("positions.len() * state_dims != states.len()")
    K = cfg.sh_coeffs()
    dev = f"cuda:{ctx.device}"
    pv = torch.empty((n, 4), dtype=torch.float32, device=dev)
    sh = torch.empty((n, K, 3), dtype=torch.float32, device=dev)
    rot = torch.empty((n, 4), dtype=torch.float32, device=dev)
    so = torch.empty((n, 4), dtype=torch.float32, device=dev)
    ctx.check(lib().npa_decode_gaussians_3d(ctx.handle, ptr(pos), ptr(st), n, state_dims,
                                            C.byref(cfg.to_c()), ptr(pv), ptr(sh), ptr(rot),
                                            ptr(so)))
    return {"position_visibility": pv, "spherical_harmonic": sh, "rotation": rot,
            "scale_opacity": so}


def splat_particles_2d(positions, colors, cfg: Splat2dConfig, ctx=None):
    """RGBA image [size*size, 4] (additive; deterministic per-pixel particle order)."""
    ctx = ctx or default_context()
    torch = _torch()
    pos = device_f32(positions, device=ctx.device).reshape(-1, 4)
    col = device_f32(colors, device=ctx.device).reshape(-1, 3)
    if col.shape[0] != pos.shape[0]:
        raise AssertionError("positions.len() != colors.len()")
    img = torch.empty((cfg.image_size * cfg.image_size, 4), dtype=torch.float32,
                      device=f"cuda:{ctx.device}")
    ctx.check(lib().npa_splat_2d(ctx.handle, ptr(pos), ptr(col), pos.shape[0],
                                 C.byref(cfg.to_c()), ptr(img)))
    return img


def splat_particles_2d_tiled(positions, colors, batch_size: int, particle_count: int,
                             cfg: Splat2dConfig, tiles_x: int, ctx=None):
    """Each of batch_size systems drawn as splat_particles_2d draws it alone, in its own
    image_size-square window (tiles_x windows per row): image [rows * size, tiles_x * size, 4]."""
    ctx = ctx or default_context()
    torch = _torch()
    pos = device_f32(positions, device=ctx.device).reshape(-1, 4)
    col = device_f32(colors, device=ctx.device).reshape(-1, 3)
    if col.shape[0] != pos.shape[0] or pos.shape[0] != batch_size * particle_count:
        raise AssertionError("positions.len() != colors.len() != batch_size * particle_count")
    rows = -(-batch_size // max(tiles_x, 1))
    img = torch.empty((rows * cfg.image_size, max(tiles_x, 1) * cfg.image_size, 4),
                      dtype=torch.float32, device=f"cuda:{ctx.device}")
    ctx.check(lib().npa_splat_2d_tiled(ctx.handle, ptr(pos), ptr(col), batch_size, particle_count,
                                       C.byref(cfg.to_c()), int(tiles_x), ptr(img)))
    return img


def _views_array(views):
    v = np.ascontiguousarray([int(x) for x in views], dtype=np.uint32)
    return v, v.ctypes.data_as(C.c_void_p)


def render_views(positions, colors, opacities, sigmas, cfg: RenderLossConfig, views=ALL_VIEWS, ctx=None):
    """project_positions + splat_projected (render_loss/projection.rs:11-29, image.rs:18-79) for
    each view: images [len(views), size, size, 5] holding r, g, b, alpha, depth_sum per pixel."""
    ctx = ctx or default_context()
    torch = _torch()
    pos = device_f32(positions, device=ctx.device).reshape(-1, 4)
    n = pos.shape[0]
    col = device_f32(colors, device=ctx.device).reshape(-1, 3)
    op = device_f32(opacities, device=ctx.device).reshape(-1)
    sg = device_f32(sigmas, device=ctx.device).reshape(-1)
    if col.shape[0] != n or op.shape[0] != n or sg.shape[0] != n:
        raise AssertionError("positions, colors, opacities and sigmas differ in length")
    varr, vptr = _views_array(views)
    img = torch.empty((len(varr), cfg.image_size, cfg.image_size, 5), dtype=torch.float32,
                      device=f"cuda:{ctx.device}")
    ctx.check(lib().npa_render_views(ctx.handle, ptr(pos), ptr(col), ptr(op), ptr(sg), n, vptr,
                                     len(varr), C.byref(cfg.to_c()), ptr(img)))
    return img


def render_attributes(states, state_dims: int, cfg: RenderLossConfig, ctx=None):
    """state_tail_render_attributes (render_loss/attributes.rs:15-87): (colors [n, 3],
    opacities [n], sigmas [n], scale_logit_derivatives [n]) on the device."""
    ctx = ctx or default_context()
    torch = _torch()
    st = device_f32(states, device=ctx.device).reshape(-1)
    if state_dims == 0 or st.numel() % state_dims:
        raise _abi.InvalidArgument(f"invalid argument: state len {st.numel()} is not divisible by "
                                   f"state_dims {state_dims}")
    n = st.numel() // state_dims
    dev = f"cuda:{ctx.device}"
    col = torch.empty((n, 3), dtype=torch.float32, device=dev)
    op, sg, dv = (torch.empty(n, dtype=torch.float32, device=dev) for _ in range(3))
    ctx.check(lib().npa_render_attributes(ctx.handle, ptr(st), n, state_dims, C.byref(cfg.to_c()),
                                          ptr(col), ptr(op), ptr(sg), ptr(dv)))
    return col, op, sg, dv


def raster_gaussians_3d(position_visibility, spherical_harmonic, rotation, scale_opacity,
                        camera: RasterCamera, ctx=None):
    """The EWA raster of oriented Gaussians (npa_raster_gaussians_3d): the frame the viewer draws
    from the planar export through bevy_gaussian_splatting (crates/bevy_automata/src/viewer/cloud.rs:80-97),
    as the published 3D Gaussian splatting forward pass. spherical_harmonic holds
    (camera.sh_degree + 1)^2 coefficients per Gaussian. Returns [height, width, 4]: premultiplied
    r, g, b and 1 - transmittance."""
    ctx = ctx or default_context()
    torch = _torch()
    pv = device_f32(position_visibility, device=ctx.device).reshape(-1, 4)
    n = pv.shape[0]
    K = (int(camera.sh_degree) + 1) ** 2
    sh = device_f32(spherical_harmonic, device=ctx.device).reshape(-1)
    rot = device_f32(rotation, device=ctx.device).reshape(-1, 4)
    so = device_f32(scale_opacity, device=ctx.device).reshape(-1, 4)
    if sh.numel() != n * K * 3 or rot.shape[0] != n or so.shape[0] != n:
        raise AssertionError("position_visibility, spherical_harmonic (K coefficients of 3), rotation "
                             "and scale_opacity differ in length")
    img = torch.empty((camera.height, camera.width, 4), dtype=torch.float32, device=f"cuda:{ctx.device}")
    ctx.check(lib().npa_raster_gaussians_3d(ctx.handle, ptr(pv), ptr(sh), ptr(rot), ptr(so), n,
                                            C.byref(camera.to_c()), ptr(img)))
    return img
