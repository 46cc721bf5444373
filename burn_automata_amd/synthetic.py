"""Seeded synthetic inputs for the benchmark configurations.

Everything is generated on the host from a counter-based generator and handed
identically to the CPU oracle and the device path, so both see the same arrays.

The generator is the reference's own ``stable_particle_uniform``
(crates/burn_automata/src/rollout/mod.rs:300-308): a SplitMix64-style mix of
(seed, stream, counter) truncated to a 24-bit uniform in [0, 1). Streams:
0 = positions, 1 = states, 2 = weights, 3 = mixture component / extra draws.

Configurations (BASELINE.json ``configs``):
  C1 ``c1``  4,096 particles, unit disk, S=16, eps=0.05, 64 steps
  C2 ``c2``  65,536 particles, unit disk, 256 steps, 512x512 splat every 32 steps
  C3 ``c3``  1,048,576 particles from an 8-component Gaussian mixture, 128 steps
  C4 ``c4``  16,384 particles on a closed 3D surface, eps=0.04, 256 steps
  C5 ``c5``  64 independent systems x 4,096 particles, bf16-rounded weights
"""
from __future__ import annotations

import math

import numpy as np

from .config import (Boundary, GaussianDecodeConfig, GaussianDecodeMode, HashGridConfig, HashGridMode,
                     NpaConfig, RasterCamera, Splat2dConfig)

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def stable_uniform(seed: int, stream: int, ids: np.ndarray) -> np.ndarray:
    """stable_particle_uniform(seed, stream, id) for an array of ids -> float64 in [0,1)."""
    with np.errstate(over="ignore"):
        ids = np.asarray(ids, dtype=np.uint64)
        v = (np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
             ^ (np.uint64(stream) * np.uint64(0x9E3779B97F4A7C15))
             ^ (ids * np.uint64(0xBF58476D1CE4E5B9)))
        v = (v ^ (v >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        v = (v ^ (v >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        v = v ^ (v >> np.uint64(31))
    return (v >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))


def _normal(seed: int, stream: int, count: int, offset: int = 0) -> np.ndarray:
    """Box-Muller standard normals from pairs of stream draws."""
    k = np.arange(offset, offset + count, dtype=np.uint64)
    u1 = np.maximum(stable_uniform(seed, stream, 2 * k), 2.0 ** -25)
    u2 = stable_uniform(seed, stream, 2 * k + np.uint64(1))
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * math.pi * u2)


def uniform_disk(count: int, seed: int = 42, radius: float = 1.0, offset: int = 0) -> np.ndarray:
    """Positions uniform in a disk: r = radius*sqrt(u1), theta = 2*pi*u2
    (the UniformCircle formula, crates/burn_automata/src/rollout/mod.rs:384-389)."""
    k = np.arange(offset, offset + count, dtype=np.uint64)
    u1 = stable_uniform(seed, 0, 2 * k)
    u2 = stable_uniform(seed, 0, 2 * k + np.uint64(1))
    r = np.sqrt(u1) * radius
    th = 2.0 * math.pi * u2
    pos = np.zeros((count, 4), dtype=np.float32)
    pos[:, 0] = (r * np.cos(th)).astype(np.float32)
    pos[:, 1] = (r * np.sin(th)).astype(np.float32)
    return pos


def uniform_ball(count: int, seed: int = 42, radius: float = 1.0) -> np.ndarray:
    """Positions uniform in a 3D ball (UniformCircle 3D branch, rollout/mod.rs:390-398)."""
    k = np.arange(count, dtype=np.uint64)
    u1 = stable_uniform(seed, 0, 3 * k)
    u2 = stable_uniform(seed, 0, 3 * k + np.uint64(1))
    u3 = stable_uniform(seed, 0, 3 * k + np.uint64(2))
    th = 2.0 * math.pi * u1
    z = 2.0 * u2 - 1.0
    rxy = np.sqrt(np.maximum(1.0 - z * z, 0.0))
    r = np.cbrt(u3) * radius
    pos = np.zeros((count, 4), dtype=np.float32)
    pos[:, 0] = (r * rxy * np.cos(th)).astype(np.float32)
    pos[:, 1] = (r * rxy * np.sin(th)).astype(np.float32)
    pos[:, 2] = (r * z).astype(np.float32)
    return pos


def normal_states(count: int, state_dims: int, seed: int = 42, std: float = 0.1,
                  offset: int = 0) -> np.ndarray:
    z = _normal(seed, 1, count * state_dims, offset * state_dims)
    return (z * std).astype(np.float32).reshape(count, state_dims)


def seeded_weights(cfg: NpaConfig, seed: int = 42, bound: float = 0.1, bf16: bool = False):
    """The NpaWeights::seeded law (crates/burn_automata/src/model.rs:29-39): w1, w2 ~ U(-0.1, 0.1),
    zero biases, drawn from the counter generator (stream 2). ``bf16`` rounds the weights to
    bfloat16 (round-to-nearest-even) and back, the C5 weight format."""
    F, H, O = cfg.perception_dims(), cfg.hidden_dims, cfg.update_dims()
    u = stable_uniform(seed, 2, np.arange(H * F + O * H, dtype=np.uint64))
    w = ((2.0 * u - 1.0) * bound).astype(np.float32)
    w1 = w[: H * F].copy()
    w2 = w[H * F:].copy()
    if bf16:
        w1 = round_bf16(w1)
        w2 = round_bf16(w2)
    return {"w1": w1, "b1": np.zeros(H, np.float32), "w2": w2, "b2": np.zeros(O, np.float32)}


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), returned as float32."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounding = np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))
    r = ((b + rounding) >> np.uint64(16)) << np.uint64(16)
    return (r & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)


def gaussian_mixture(count: int, seed: int = 42, components: int = 8) -> np.ndarray:
    """C3: isotropic 8-component mixture, equal weights, sigma_k = 0.02 * 10**(k/7),
    means uniform in [-0.6, 0.6]^2."""
    kk = np.arange(components, dtype=np.uint64)
    means = np.stack([stable_uniform(seed, 3, 2 * kk), stable_uniform(seed, 3, 2 * kk + np.uint64(1))],
                     axis=1) * 1.2 - 0.6
    sig = 0.02 * 10.0 ** (np.arange(components) / (components - 1))
    ids = np.arange(count, dtype=np.uint64)
    comp = np.minimum((stable_uniform(seed, 3, ids + np.uint64(1000)) * components).astype(np.int64),
                      components - 1)
    zx = _normal(seed, 0, count, 0)
    zy = _normal(seed, 0, count, count)
    pos = np.zeros((count, 4), dtype=np.float32)
    pos[:, 0] = (means[comp, 0] + sig[comp] * zx).astype(np.float32)
    pos[:, 1] = (means[comp, 1] + sig[comp] * zy).astype(np.float32)
    return pos


def closed_surface_3d(count: int, seed: int = 42) -> np.ndarray:
    """C4 geometry: an ellipsoid (semi-axes 0.6, 0.45, 0.35) joined by a handle
    (a half torus, major radius 0.32, minor 0.07, arching over +z), triangulated
    (~20k triangles) and sampled uniformly by area."""
    tris = _surface_triangles()
    a = tris[:, 1] - tris[:, 0]
    b = tris[:, 2] - tris[:, 0]
    area = 0.5 * np.linalg.norm(np.cross(a, b), axis=1)
    cdf = np.cumsum(area)
    cdf /= cdf[-1]
    ids = np.arange(count, dtype=np.uint64)
    t = np.searchsorted(cdf, stable_uniform(seed, 0, 3 * ids), side="right")
    t = np.minimum(t, len(tris) - 1)
    r1 = np.sqrt(stable_uniform(seed, 0, 3 * ids + np.uint64(1)))
    r2 = stable_uniform(seed, 0, 3 * ids + np.uint64(2))
    p = ((1 - r1)[:, None] * tris[t, 0] + (r1 * (1 - r2))[:, None] * tris[t, 1]
         + (r1 * r2)[:, None] * tris[t, 2])
    pos = np.zeros((count, 4), dtype=np.float32)
    pos[:, :3] = p.astype(np.float32)
    return pos


def _surface_triangles() -> np.ndarray:
    def grid_tris(fn, nu, nv, wrap_u, wrap_v):
        us = np.linspace(0, 1, nu + (0 if wrap_u else 1), endpoint=not wrap_u)
        vs = np.linspace(0, 1, nv + (0 if wrap_v else 1), endpoint=not wrap_v)
        P = fn(us[:, None], vs[None, :])
        iu = len(us) if wrap_u else len(us) - 1
        iv = len(vs) if wrap_v else len(vs) - 1
        out = []
        for i in range(iu):
            i2 = (i + 1) % len(us)
            for j in range(iv):
                j2 = (j + 1) % len(vs)
                out.append((P[i, j], P[i2, j], P[i2, j2]))
                out.append((P[i, j], P[i2, j2], P[i, j2]))
        return np.array(out)

    def ellipsoid(u, v):
        th = u * 2 * math.pi
        ph = v * math.pi
        return np.stack(np.broadcast_arrays(0.6 * np.sin(ph) * np.cos(th), 0.45 * np.sin(ph) * np.sin(th),
                                            0.35 * np.cos(ph)), axis=-1)

    def handle(u, v):
        al = u * math.pi  # half circle over the top
        be = v * 2 * math.pi
        R, r = 0.32, 0.07
        cx = (R + r * np.cos(be)) * np.cos(al)
        cz = 0.2 + (R + r * np.cos(be)) * np.sin(al)
        cy = r * np.sin(be)
        return np.stack(np.broadcast_arrays(cx, cy, cz), axis=-1)

    t1 = grid_tris(ellipsoid, 100, 70, True, False)
    t2 = grid_tris(handle, 60, 24, False, True)
    return np.concatenate([t1, t2], axis=0)


def config_c1(particles: int = 4096, seed: int = 42):
    """C1/C2 model and grid: growing_2d NpaConfig with S=16, H=128, eps=eps0=0.05, density_grad off
    (F=64, O=18) on a Particle-mode 64x64 Clamped hashgrid."""
    model = NpaConfig.growing_2d().replace(eps0=0.05, density_grad=False)
    grid = HashGridConfig(2, Boundary.Clamped, HashGridMode.Particle, (64, 64, 1), 0.05, 32)
    return model, grid


def workload(name: str, seed: int = 42, particles: int | None = None):
    """Returns dict(model, grid, batch, n, positions, states, weights, steps, decode_every, splat)."""
    name = name.lower()
    if name in ("c1", "c2", "c1_dgrad"):
        n = particles or (4096 if name != "c2" else 65536)
        model, grid = config_c1(n, seed)
        if name == "c1_dgrad":
            model = model.replace(density_grad=True)
        steps = 256 if name == "c2" else 64
        out = dict(model=model, grid=grid, batch=1, n=n, positions=uniform_disk(n, seed),
                   states=normal_states(n, model.state_dims, seed),
                   weights=seeded_weights(model, seed), steps=steps, dt=1.0, update_prob=0.5,
                   seed=seed)
        if name == "c2":
            out["decode_every"] = 32
            out["splat"] = Splat2dConfig(image_size=512, sigma=0.004 * 511 / 2, lo=-1.0, hi=1.0,
                                         normalize_color=True, y_up=True, pixel_size=2.0 / 512)
        return out
    if name == "c3":
        n = particles or 1 << 20
        model, grid = config_c1(n, seed)
        return dict(model=model, grid=grid, batch=1, n=n, positions=gaussian_mixture(n, seed),
                    states=normal_states(n, model.state_dims, seed),
                    weights=seeded_weights(model, seed), steps=128, dt=1.0, update_prob=0.5,
                    seed=seed)
    if name == "c4":
        n = particles or 16384
        model = NpaConfig.growing_3dgs().replace(state_dims=16, hidden_dims=128, eps0=0.04,
                                                 density_grad=False, alpha=0.5)
        grid = HashGridConfig(3, Boundary.Clamped, HashGridMode.Particle, (32, 32, 32), 0.04, 64)
        # decode: oriented Gaussians (gaussian.rs:53-223) drawn by the EWA raster of oriented
        # Gaussians at 512x512 (npa_state_raster_gaussians_3d: the viewer's draw of the decode),
        # from a fixed camera framing the surface (extent about 1.2 x 0.9 x 1.1 around the origin)
        return dict(model=model, grid=grid, batch=1, n=n, positions=closed_surface_3d(n, seed),
                    states=normal_states(n, model.state_dims, seed),
                    weights=seeded_weights(model, seed), steps=256, dt=1.0, update_prob=0.5,
                    seed=seed, decode_every=32,
                    decode=GaussianDecodeConfig(mode=GaussianDecodeMode.GaussianSh0Oriented),
                    camera=RasterCamera.look_at((0.9, 1.2, 2.6), (0.0, 0.0, 0.1), width=512, height=512))
    if name == "c5":
        n = particles or 4096
        b = 64
        model, grid = config_c1(n, seed)
        pos = np.concatenate([uniform_disk(n, seed, offset=k * n) for k in range(b)], axis=0)
        # decode at steps 64 and 256: each system in a 128x128 window of a 1024x1024 image
        return dict(model=model, grid=grid, batch=b, n=n, positions=pos,
                    states=normal_states(b * n, model.state_dims, seed),
                    weights=seeded_weights(model, seed, bf16=True), steps=256, dt=1.0,
                    update_prob=0.5, seed=seed, decode_steps=(64, 256), tiles_x=8,
                    splat=Splat2dConfig(image_size=128, sigma=0.004 * 127 / 2, lo=-1.0, hi=1.0,
                                        normalize_color=True, y_up=True, pixel_size=2.0 / 128))
    raise ValueError(f"unknown workload {name!r}")
