"""CPU checks that pin the oracle (oracle/libnpa_oracle.so) to the reference's behaviour.

The reference path is Rust and cannot be built here, so the oracle is a C restatement. These
tests pin it with, in order of strength:
  * the reference's own known-answer unit tests for this path (values transcribed into
    tests/golden/reference_known_answers.json, each with its file:line);
  * integer closed forms restated from the reference source in a second language (cell hash,
    mask hash), brute force on small inputs (counting sort, neighbour sets and order, density,
    blur), and float64 closed forms (poly6/spiky constants, log-normalisation, equivariance
    scales, motion, splat of one particle);
  * invariants the mathematics fixes: the moment-corrected SPH gradient of a linear field is the
    field's slope for every particle with an invertible moment matrix, rigid scale equivariance
    of a scale-equivariant model (crates/burn_automata/tests/core/equivariance.rs:4-67),
    composition (step == perceive -> MLP -> Euler; rollout == repeated masked steps), additivity
    of the splat.
Each check is chosen so that a plausible slip (a dropped term, a swapped sign, a transposed
operand, a wrong index or order) fails it.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import (Boundary, EquivarianceMode, GaussianDecodeConfig,
                                      GaussianDecodeMode, HashGridConfig, HashGridMode, NpaConfig,
                                      PerceptionOptions, Splat2dConfig)
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
KNOWN = json.load(open(os.path.join(HERE, "golden", "reference_known_answers.json")))

M32 = 0xFFFFFFFF
f32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _built():
    O.build()
    O.lib()


# --------------------------------------------------------------------------------------------
# independent restatements (integer closed forms; float32 evaluation order as in the reference)
# --------------------------------------------------------------------------------------------

def mix_coord(value: int, salt: int) -> int:
    """hashgrid.rs:157-165: (value as i32 as u32) ^ salt, then xorshift-multiply."""
    x = (value & M32) ^ salt
    x ^= x >> 16
    x = (x * 0x7FEB352D) & M32
    x ^= x >> 15
    x = (x * 0x846CA68B) & M32
    x ^= x >> 16
    return x


def cell_coords_ref(p, cfg: HashGridConfig):
    """cell_coords_for_position (hashgrid.rs:98-121) in float32."""
    out = [0, 0, 0]
    eps = f32(cfg.eps)
    for a in range(cfg.dim):
        x = f32(p[a])
        if cfg.mode == HashGridMode.Particle:
            out[a] = int(math.floor(float(x / eps)))
            continue
        size = int(cfg.grid_size[a])
        extent = eps * f32(size)
        half = extent * f32(0.5)
        c = int(math.floor(float((x + half) / eps)))
        c = c % size if cfg.boundary == Boundary.Periodic else min(max(c, 0), size - 1)
        out[a] = c
    return tuple(out)


def cell_index_ref(coords, cfg: HashGridConfig):
    """cell_index_from_coords / particle_cell_hash (hashgrid.rs:123-155)."""
    if cfg.mode == HashGridMode.Particle:
        h = mix_coord(coords[0], 0x9E3779B9) ^ mix_coord(coords[1], 0x85EBCA6B)
        if cfg.dim == 3:
            h ^= mix_coord(coords[2], 0xC2B2AE35)
        return h % cfg.cell_count()
    stride, h = 1, 0
    for a in range(cfg.dim):
        size = int(cfg.grid_size[a])
        c = coords[a]
        if cfg.boundary == Boundary.Periodic:
            c %= size
        elif c < 0 or c >= size:
            return None
        h += c * stride
        stride *= size
    return h


def hash_u32_ref(v: int) -> int:
    """hash_u32 of the reference's CPU replica of the device mask
    (crates/burn_automata/tests/gpu_wgpu/common.rs:126-133)."""
    x = v & M32
    x = (x ^ 61) ^ (x >> 16)
    x = (x + (x << 3)) & M32
    x ^= x >> 4
    x = (x * 0x27D4EB2D) & M32
    return x ^ (x >> 15)


def random01_ref(particle: int, step: int, seed: int) -> float:
    """gpu_random01 (common.rs:121-124)."""
    mixed = hash_u32_ref(particle ^ hash_u32_ref((step + 0x9E3779B9) & M32) ^ seed)
    return float(f32(mixed >> 8) * f32(1.0 / 16777216.0))


def pair_table(pos: np.ndarray, cfg: HashGridConfig):
    """All-pairs delta / r^2 in float32 with the reference's operation order
    (neighbor_delta hashgrid.rs:167-181; r2 = sum of squares from 0, neighbor.rs:35-37)."""
    d = cfg.dim
    P = pos[:, :d].astype(f32)
    D = P[None, :, :] - P[:, None, :]  # D[i, j] = p_j - p_i
    if cfg.boundary == Boundary.Periodic:
        for a in range(d):
            extent = f32(cfg.grid_size[a]) * f32(cfg.eps)
            half = extent * f32(0.5)
            col = D[:, :, a]
            col = np.where(col > half, col - extent, np.where(col < -half, col + extent, col))
            D[:, :, a] = col
    r2 = np.zeros(D.shape[:2], f32)
    for a in range(d):
        r2 = r2 + D[:, :, a] * D[:, :, a]
    return D, r2


def eps2(cfg):
    return f32(cfg.eps) * f32(cfg.eps)


def k6(cfg):
    """smoothing_poly6_normalization (kernels.rs:126-132), float64."""
    e = float(cfg.eps)
    return 4.0 / (math.pi * e ** 8) if cfg.dim == 2 else 315.0 / (64.0 * math.pi * e ** 9)


def k5(cfg):
    """gradient_spiky_normalization (kernels.rs:134-140), float64."""
    e = float(cfg.eps)
    return 10.0 / (math.pi * e ** 5) if cfg.dim == 2 else 15.0 / (math.pi * e ** 6)


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30)) if b.size else 0.0


def _grids():
    g2 = HashGridConfig.growing_2d().replace(eps=0.05, grid_size=(64, 64, 1))
    return {
        "particle2d": g2,
        "particle2d_small_table": g2.replace(grid_size=(4, 4, 1)),  # many hash collisions
        "grid2d_clamped": HashGridConfig(2, Boundary.Clamped, HashGridMode.Grid, (24, 20, 1), 0.08),
        "grid2d_periodic": HashGridConfig(2, Boundary.Periodic, HashGridMode.Grid, (16, 12, 1), 0.1),
        "particle3d": HashGridConfig.growing_3dgs().replace(eps=0.2, grid_size=(8, 8, 8)),
        "grid3d_periodic": HashGridConfig(3, Boundary.Periodic, HashGridMode.Grid, (8, 6, 5), 0.25),
    }


def _positions(name, cfg, n, seed=7):
    rng = np.random.default_rng(seed)
    d = cfg.dim
    pos = np.zeros((n, 4), f32)
    if cfg.mode == HashGridMode.Grid and cfg.boundary == Boundary.Periodic:
        for a in range(d):
            half = cfg.grid_size[a] * cfg.eps / 2
            pos[:, a] = rng.uniform(-half, half, n)
    else:
        pos[:, :d] = rng.uniform(-0.6, 0.6, (n, d))
        pos[: n // 10, :d] *= 2.5  # some outside a clamped grid / far from the origin
    return pos


# --------------------------------------------------------------------------------------------
# hashgrid
# --------------------------------------------------------------------------------------------

@pytest.mark.parametrize("name", list(_grids()))
def test_cell_hash_matches_integer_restatement(name):
    cfg = _grids()[name]
    pos = _positions(name, cfg, 400)
    extra = np.array([[-1e-9, 0.0, 0.0, 0.0], [0.0, -0.0, 0.0, 0.0],
                      [cfg.eps, -cfg.eps, cfg.eps, 0.0], [123.4, -77.7, 5.5, 0.0]], f32)
    for p in np.concatenate([pos, extra]):
        coords = cell_coords_ref(p, cfg)
        assert O.cell_coords(p, cfg)[: cfg.dim] == coords[: cfg.dim]
        idx = cell_index_ref(coords, cfg)
        assert O.cell_for_position(p, cfg) == idx


def test_hashgrid_counts_particles_per_cell():
    """hashgrid_counts_particles_per_cell (crates/burn_automata_kernels/src/lib.rs:73-84)."""
    ka = KNOWN["hashgrid_counts_particles_per_cell"]
    cfg = HashGridConfig.growing_2d().replace(grid_size=tuple(ka["grid_size"]))
    g = O.build_hashgrid(np.array(ka["positions"], f32), 1, 2, cfg)
    assert len(g.bin_offsets) == cfg.cell_count() + 1
    assert len(g.permutation) == 2
    assert np.any(np.diff(g.bin_offsets.astype(np.int64)) > 0)


@pytest.mark.parametrize("name", list(_grids()))
@pytest.mark.parametrize("batch", [1, 3])
def test_hashgrid_is_a_stable_counting_sort(name, batch):
    cfg = _grids()[name]
    n = 300
    pos = np.concatenate([_positions(name, cfg, n, seed=11 + b) for b in range(batch)])
    g = O.build_hashgrid(pos, batch, n, cfg)
    C = cfg.cell_count()
    cells = np.array([cell_index_ref(cell_coords_ref(p, cfg), cfg) for p in pos], np.int64)
    assert g.bin_offsets[0] == 0 and g.bin_offsets[-1] == batch * n
    for b in range(batch):
        cb = cells[b * n:(b + 1) * n]
        counts = np.bincount(cb, minlength=C)
        want_off = b * n + np.concatenate([[0], np.cumsum(counts)])
        np.testing.assert_array_equal(g.bin_offsets[b * C:(b + 1) * C + 1], want_off)
        order = np.argsort(cb, kind="stable")  # stable: original order within a bin
        np.testing.assert_array_equal(g.permutation[b * n:(b + 1) * n], order)
        inv = g.inverse_permutation[b * n:(b + 1) * n]
        np.testing.assert_array_equal(inv[order], np.arange(n))


def test_hashgrid_rejects_invalid_configs():
    """validate (crates/burn_automata_kernels/src/config.rs:66-99) error variants."""
    from burn_automata_amd import _abi
    pos = np.zeros((2, 4), f32)
    good = HashGridConfig.growing_2d()
    cases = [
        (good.replace(dim=4), _abi.InvalidDim),
        (good.replace(eps=0.0), _abi.InvalidEps),
        (good.replace(eps=float("nan")), _abi.InvalidEps),
        (good.replace(grid_size=(0, 64, 1)), _abi.InvalidGridSize),
        (good.replace(grid_size=(48, 64, 1)), _abi.ParticleModeRequiresPowerOfTwo),
    ]
    for cfg, err in cases:
        with pytest.raises(err):
            O.build_hashgrid(pos, 1, 2, cfg)
    with pytest.raises(_abi.PositionShape):
        O.build_hashgrid(pos, 1, 3, good)


# --------------------------------------------------------------------------------------------
# neighbour lists
# --------------------------------------------------------------------------------------------

def _offset_order(dim):
    zs = (-1, 0, 1) if dim == 3 else (0,)
    return [(dx, dy, dz) for dz in zs for dy in (-1, 0, 1) for dx in (-1, 0, 1)]


@pytest.mark.parametrize("name", list(_grids()))
def test_neighbor_lists_match_brute_force_sets_and_order(name):
    cfg = _grids()[name]
    n = 500 if cfg.dim == 2 else 300
    batch = 2
    pos = np.concatenate([_positions(name, cfg, n, seed=21 + b) for b in range(batch)])
    off, idx = O.neighbor_lists(pos, batch, n, cfg)
    g = O.build_hashgrid(pos, batch, n, cfg)
    offsets = _offset_order(cfg.dim)
    total_pairs = 0
    for b in range(batch):
        P = pos[b * n:(b + 1) * n]
        _, r2 = pair_table(P, cfg)
        coords = [cell_coords_ref(p, cfg) for p in P]
        inv = g.inverse_permutation[b * n:(b + 1) * n]
        for i in range(n):
            js = np.nonzero(r2[i] < eps2(cfg))[0]
            keys = []
            for j in js:
                rel_c = []
                for a in range(3 if cfg.dim == 3 else 2):
                    dc = coords[j][a] - coords[i][a]
                    if cfg.mode == HashGridMode.Grid and cfg.boundary == Boundary.Periodic:
                        size = cfg.grid_size[a]
                        dc = (dc + 1) % size - 1
                    rel_c.append(dc)
                if cfg.dim == 2:
                    rel_c.append(0)
                keys.append((offsets.index(tuple(rel_c)), int(inv[j]), int(j)))
            want = [b * n + k[2] for k in sorted(keys)]
            got = idx[off[b * n + i]:off[b * n + i + 1]].tolist()
            assert got == want, (name, b, i)
            total_pairs += len(want)
    assert total_pairs > 2 * batch * n  # the fixture has real neighbourhoods


def test_pair_at_exactly_eps_is_not_a_neighbour():
    """Acceptance is r^2 < eps^2, strict (neighbor.rs:35-37): a pair exactly eps apart in float32
    (delta = eps, so r^2 == eps^2 bit for bit) is not a neighbour."""
    for mode in (HashGridMode.Particle, HashGridMode.Grid):
        cfg = HashGridConfig(2, Boundary.Clamped, mode, (16, 16, 1), 0.05)
        pos = np.array([[0.0, 0.0, 0, 0], [0.05, 0.0, 0, 0], [0.0, -0.05, 0, 0]], f32)
        _, r2 = pair_table(pos, cfg)
        assert r2[0, 1] == eps2(cfg) and r2[0, 2] == eps2(cfg)
        off, idx = O.neighbor_lists(pos, 1, 3, cfg)
        assert idx.tolist() == [0, 1, 2]  # each particle sees only itself
        out = O.perceive_with_options(pos, np.zeros((3, 1), f32), 1, 3, 1, cfg, _opts(eps0=0.05))
        assert out.density == pytest.approx([k6(cfg) * 0.05 ** 6] * 3, rel=1e-6)


def test_neighbor_search_counts_match_reference_fixture():
    """Exact pair count of spatial_strategy_bvh_matches_hashgrid_neighbor_counts
    (crates/burn_automata_kernels/src/lib.rs:530-564) by brute force: the hashgrid walk must
    find every pair within eps and nothing else."""
    ka = KNOWN["spatial_strategy_bvh_matches_hashgrid_neighbor_counts"]
    cfg = HashGridConfig.growing_3dgs().replace(grid_size=tuple(ka["grid_size"]))
    pos = np.array(ka["positions"], f32)
    off, idx = O.neighbor_lists(pos, 1, len(pos), cfg)
    _, r2 = pair_table(pos, cfg)
    assert len(idx) == int(np.sum(r2 < eps2(cfg)))


# --------------------------------------------------------------------------------------------
# SPH perception
# --------------------------------------------------------------------------------------------

def test_perceive_matches_upstream_sph_kernel_constants():
    """perceive_matches_upstream_sph_kernel_constants (lib.rs:100-120), plus the same numbers
    derived by hand from K6 = 4/(pi eps^8), K5 = 10/(pi eps^5)."""
    ka = KNOWN["perceive_matches_upstream_sph_kernel_constants"]
    cfg = HashGridConfig.growing_2d().replace(grid_size=tuple(ka["grid_size"]), eps=ka["eps"])
    pos = np.array(ka["positions"], f32)
    st = np.array(ka["states"], f32)
    out = O.perceive(pos, st, 1, 2, 2, cfg, True, True)
    for key, index, want, tol in ka["expect"]:
        got = getattr(out, key).reshape(-1)[index]
        assert abs(float(got) - want) <= tol, (key, index, got, want)
    # closed forms in float64
    e, r = float(cfg.eps), 0.05
    rho = k6(cfg) * (e ** 6 + (e * e - r * r) ** 3)
    w0, w1 = k6(cfg) * e ** 6, k6(cfg) * (e * e - r * r) ** 3
    grad_mag = k5(cfg) * 3.0 * (e - r) ** 2 / r
    assert out.density == pytest.approx([rho, rho], rel=2e-6)
    assert out.blurred_state.reshape(-1) == pytest.approx(
        [w0 / rho, w1 / rho, w1 / rho, w0 / rho], rel=2e-6)
    # two particles: rank-1 moment matrix -> identity correction; scale eps/eps0 = 1
    vol = 1.0 / rho
    sg = out.state_gradient.reshape(2, 2, 2)  # [particle][channel][axis]
    assert sg[0, 0, 0] == pytest.approx((0.0 - 1.0) * vol * grad_mag * r, rel=2e-6)
    assert sg[0, 1, 0] == pytest.approx((1.0 - 0.0) * vol * grad_mag * r, rel=2e-6)
    assert sg[1, 0, 0] == pytest.approx((1.0 - 0.0) * vol * grad_mag * (-r), rel=2e-6)
    dg = out.density_gradient.reshape(2, 2)
    assert dg[0, 0] == pytest.approx(grad_mag * r / 2, rel=2e-6)  # x (eps/eps0)^3 / N
    assert dg[1, 0] == pytest.approx(-grad_mag * r / 2, rel=2e-6)
    assert np.all(sg[:, :, 1] == 0) and np.all(dg[:, 1] == 0)


def test_perceive_returns_finite_reference_features():
    """perceive_returns_finite_reference_features (lib.rs:87-97)."""
    ka = KNOWN["perceive_returns_finite_reference_features"]
    cfg = HashGridConfig.growing_2d()
    out = O.perceive(np.array(ka["positions"], f32), np.array(ka["states"], f32), 1, 2, 2, cfg,
                     True, True)
    assert out.feature_dims == 2 * 2 + 2 * cfg.dim + cfg.dim
    assert out.features.size == 2 * out.feature_dims
    assert np.all(np.isfinite(out.features))
    assert np.all(out.density > 0)


def _opts(**kw):
    o = PerceptionOptions.new(True, True, kw.pop("eps0", 0.05))
    for k, v in kw.items():
        setattr(o, k, v)
    return o


@pytest.mark.parametrize("name", ["particle2d", "grid2d_periodic", "particle3d"])
def test_density_and_blur_match_brute_force(name):
    cfg = _grids()[name]
    n, S = (600, 3) if cfg.dim == 2 else (400, 3)
    pos = _positions(name, cfg, n, seed=5)
    rng = np.random.default_rng(3)
    st = rng.normal(0, 1, (n, S)).astype(f32)
    out = O.perceive_with_options(pos, st, 1, n, S, cfg, _opts(eps0=cfg.eps))
    _, r2 = pair_table(pos, cfg)
    inside = r2 < eps2(cfg)
    W = np.where(inside, k6(cfg) * (float(cfg.eps) ** 2 - r2.astype(np.float64)) ** 3, 0.0)
    rho = W.sum(axis=1)
    assert rel(out.density, rho) < 2e-6
    # blur uses the oracle's own float32 density for the volume (isolates the blur sum)
    vol = 1.0 / out.density.astype(np.float64)
    blur = W @ (st.astype(np.float64) * vol[:, None])
    assert rel(out.blurred_state, blur) < 2e-5


def _linear_field_case(dim, S=4, h=None, eps=0.06, seed=0):
    rng = np.random.default_rng(seed)
    h = h or eps / 3.2
    ax = np.arange(-0.5, 0.5, h)
    grids = np.meshgrid(*([ax] * dim), indexing="ij")
    P = np.stack([g.reshape(-1) for g in grids], axis=1)
    P += rng.uniform(-0.3 * h, 0.3 * h, P.shape)
    n = P.shape[0]
    pos = np.zeros((n, 4), f32)
    pos[:, :dim] = P
    A = rng.uniform(-2, 2, (S, dim))
    b = rng.uniform(-1, 1, S)
    st = (pos[:, :dim].astype(np.float64) @ A.T + b).astype(f32)
    interior = np.all(np.abs(P) < 0.5 - 1.5 * eps, axis=1)
    return pos, st, A, interior


@pytest.mark.parametrize("dim", [2, 3])
def test_moment_corrected_gradient_of_a_linear_field_is_its_slope(dim):
    """M = sum_j d (x) gradW_j V_j and g = sum_j (s_j - s_i) gradW_j V_j = a^T M for s = a.x,
    so the hybrid gradient g M^-1 (normalize.rs:93-118) returns a for every particle with an
    invertible M; without the correction the jittered lattice is off by a few percent."""
    eps = 0.06 if dim == 2 else 0.12
    pos, st, A, interior = _linear_field_case(dim, eps=eps, h=eps / (3.2 if dim == 2 else 2.2))
    n, S = st.shape
    if dim == 2:
        cfg = HashGridConfig.growing_2d().replace(eps=eps, grid_size=(64, 64, 1))
    else:
        cfg = HashGridConfig.growing_3dgs().replace(eps=eps, grid_size=(16, 16, 16))
    out = O.perceive_with_options(pos, st, 1, n, S, cfg, _opts(eps0=eps, density_grad=False))
    g = out.state_gradient.reshape(n, S, dim)[interior]
    assert interior.sum() > 50
    want = np.broadcast_to(A, g.shape)
    assert rel(g, want) < 2e-3
    raw = O.perceive_with_options(pos, st, 1, n, S, cfg,
                                  _opts(eps0=eps, density_grad=False, hybrid_state_gradient=False))
    assert rel(raw.state_gradient.reshape(n, S, dim)[interior], want) > 1e-2


def _log_norm(v):
    """log_normalize_vector (normalize.rs:60-69) in float64."""
    nrm = np.maximum(np.sqrt(np.sum(v * v, axis=-1, keepdims=True) + 1e-12), 1e-6)
    return v * np.log1p(nrm) / nrm


def test_gradient_scaling_and_log_normalisation_closed_forms():
    """normalize_state_gradient / normalize_density_gradient (normalize.rs:5-58): state gradient
    x eps/eps0, density gradient x (eps/eps0)^(1+d) / N, each followed by the per-vector
    log-normalisation v ln1p(n)/n."""
    cfg = _grids()["particle2d"]
    n, S, d = 700, 3, 2
    pos = _positions("particle2d", cfg, n, seed=9)
    st = np.random.default_rng(1).normal(0, 0.5, (n, S)).astype(f32)
    eps0 = 0.035
    base = O.perceive_with_options(pos, st, 1, n, S, cfg, _opts(
        eps0=eps0, scale_equivariance=False, particle_density_equivariance=False))
    scaled = O.perceive_with_options(pos, st, 1, n, S, cfg, _opts(eps0=eps0))
    logn = O.perceive_with_options(pos, st, 1, n, S, cfg, _opts(
        eps0=eps0, log_norm_grad=True, log_norm_density_grad=True))
    s = cfg.eps / eps0
    sg0 = base.state_gradient.astype(np.float64).reshape(n, S, d)
    dg0 = base.density_gradient.astype(np.float64).reshape(n, d)
    assert rel(scaled.state_gradient.reshape(n, S, d), sg0 * s) < 1e-6
    assert rel(scaled.density_gradient.reshape(n, d), dg0 * s ** (1 + d) / n) < 1e-6
    assert rel(logn.state_gradient.reshape(n, S, d), _log_norm(sg0 * s)) < 1e-5
    assert rel(logn.density_gradient.reshape(n, d), _log_norm(dg0 * s ** (1 + d) / n)) < 1e-5
    # density, blur untouched by the options
    np.testing.assert_array_equal(base.density, logn.density)
    np.testing.assert_array_equal(base.blurred_state, logn.blurred_state)


def test_log_normalisation_of_small_vectors_uses_log1p():
    """log_normalize_vector calls ln_1p (normalize.rs:65): for gradient norms of 1e-7..1e-4 the
    scale ln1p(n)/n is 1 - n/2 + ..., which log(1 + n) in float32 cannot resolve."""
    cfg = _grids()["particle2d"]
    n, S, d = 500, 2, 2
    pos = _positions("particle2d", cfg, n, seed=12)
    st = (np.random.default_rng(5).normal(0, 1, (n, S)) * np.array([1e-8, 3e-7])).astype(f32)
    base = O.perceive_with_options(pos, st, 1, n, S, cfg, _opts(eps0=0.05, density_grad=False))
    logn = O.perceive_with_options(pos, st, 1, n, S, cfg, _opts(
        eps0=0.05, density_grad=False, log_norm_grad=True))
    g = base.state_gradient.astype(np.float64).reshape(n, S, d)
    nrm = np.sqrt(np.sum(g * g, axis=-1))
    assert np.median(nrm) < 1e-4 and np.median(nrm) > 1e-7
    want = _log_norm(g)
    got = logn.state_gradient.reshape(n, S, d).astype(np.float64)
    nz = want != 0
    assert np.max(np.abs(got[nz] - want[nz]) / np.abs(want[nz])) < 3e-6


@pytest.mark.parametrize("dgrad,posf", [(False, False), (True, False), (True, True)])
def test_feature_row_layout(dgrad, posf):
    """Feature row = [state, blur, state gradient (channel-major), density gradient?, position?]
    (forward.rs:100-133; width crates/burn_automata/src/config.rs:133-139)."""
    cfg = _grids()["particle2d"]
    n, S, d = 300, 4, 2
    pos = _positions("particle2d", cfg, n, seed=2)
    st = np.random.default_rng(4).normal(0, 1, (n, S)).astype(f32)
    out = O.perceive_with_options(pos, st, 1, n, S, cfg,
                                  _opts(eps0=0.05, density_grad=dgrad, position_features=posf))
    F = 2 * S + S * d + d * dgrad + d * posf
    assert out.feature_dims == F and out.features.shape == (n, F)
    f = out.features
    np.testing.assert_array_equal(f[:, :S], st)
    np.testing.assert_array_equal(f[:, S:2 * S], out.blurred_state)
    np.testing.assert_array_equal(f[:, 2 * S:2 * S + S * d], out.state_gradient.reshape(n, -1))
    c = 2 * S + S * d
    if dgrad:
        np.testing.assert_array_equal(f[:, c:c + d], out.density_gradient.reshape(n, d))
        c += d
    if posf:
        np.testing.assert_array_equal(f[:, c:c + d], pos[:, :d])


# --------------------------------------------------------------------------------------------
# update MLP, motion, Euler
# --------------------------------------------------------------------------------------------

def _int_model(S=4, H=16, d=2, dgrad=False):
    m = NpaConfig.growing_2d().replace(state_dims=S, hidden_dims=H, density_grad=dgrad, eps0=0.05)
    F, Oo = m.perception_dims(), m.update_dims()
    rng = np.random.default_rng(8)
    w = {"w1": rng.integers(-3, 4, (H, F)).astype(f32), "b1": rng.integers(-5, 6, H).astype(f32),
         "w2": rng.integers(-3, 4, (Oo, H)).astype(f32), "b2": rng.integers(-5, 6, Oo).astype(f32)}
    return m, w


def test_mlp_with_integer_weights_is_exact():
    """forward_update_from_features (crates/burn_automata/src/model.rs:900-940): h = ReLU(b1 +
    W1 f), u = b2 + W2 h. With small integers every partial sum is exact in float32."""
    m, w = _int_model()
    F = m.perception_dims()
    feats = np.random.default_rng(0).integers(-4, 5, (257, F)).astype(f32)
    h = np.maximum(feats.astype(np.int64) @ w["w1"].astype(np.int64).T + w["b1"].astype(np.int64), 0)
    u = h @ w["w2"].astype(np.int64).T + w["b2"].astype(np.int64)
    assert np.any(feats.astype(np.int64) @ w["w1"].astype(np.int64).T + w["b1"] < 0)  # ReLU active
    got = O.forward_update_from_features(m, w, feats)
    np.testing.assert_array_equal(got, u.astype(f32))


@pytest.mark.parametrize("equiv", [EquivarianceMode.ParticleDensityAndScale,
                                   EquivarianceMode.NoEquivariance])
def test_motion_is_alpha_u_eps_over_one_plus_norm(equiv):
    """forward_from_features_with_eps (model.rs:867-898) with motion_eps (config.rs:156-162)."""
    m, w = _int_model()
    m = m.replace(equivariance=equiv, alpha=0.37)
    F, d, S = m.perception_dims(), 2, m.state_dims
    feats = np.random.default_rng(1).integers(-4, 5, (64, F)).astype(f32)
    u = O.forward_update_from_features(m, w, feats).astype(np.float64)
    eps = 0.081
    dx, ds = O.forward_from_features_with_eps(m, w, feats, eps)
    meps = eps if equiv == EquivarianceMode.ParticleDensityAndScale else m.eps0
    nrm = np.sqrt(np.sum(u[:, :d] ** 2, axis=1, keepdims=True))
    assert rel(dx[:, :d], 0.37 * u[:, :d] * meps / (1 + nrm)) < 1e-6
    assert np.all(dx[:, d:] == 0)
    np.testing.assert_array_equal(ds, u[:, d:].astype(f32))


def test_euler_step_applies_masks_and_boundaries():
    """euler_step_applies_masks_and_boundaries (lib.rs:359-383)."""
    ka = KNOWN["euler_step_applies_masks_and_boundaries"]
    cfg = HashGridConfig.growing_2d()
    npos, nst = O.euler_step(np.array(ka["positions"], f32), np.array(ka["states"], f32),
                             np.array(ka["dx"], f32), np.array(ka["ds"], f32), 1, 2, 1, cfg, 1.0,
                             np.array(ka["mask"], f32))
    assert npos[0, 0] == ka["expect_pos0_x"] and npos[1, 0] == ka["expect_pos1_x"]
    assert nst.reshape(-1).tolist() == ka["expect_states"]


def test_euler_step_clamps_3d_opacity_logit():
    """euler_step_clamps_3d_opacity_logit (lib.rs:386-403)."""
    ka = KNOWN["euler_step_clamps_3d_opacity_logit"]
    cfg = HashGridConfig.growing_3dgs()
    for case in ka["cases"]:
        _, nst = O.euler_step(np.zeros((1, 4), f32), np.array(case["states"], f32),
                              np.zeros((1, 4), f32), np.array(case["ds"], f32), 1, 1, 4, cfg, 1.0)
        assert nst.reshape(-1)[3] == case["expect_channel3"]


def test_euler_closed_forms():
    """p + dt dx m over spatial_mem_dims axes (4 in 3D), periodic wrap, s + dt ds m
    (step.rs:4-55; wrap_position hashgrid.rs:183-193)."""
    rng = np.random.default_rng(3)
    n, S = 50, 5
    pos = rng.uniform(-0.9, 0.9, (n, 4)).astype(f32)
    st = rng.normal(0, 1, (n, S)).astype(f32)
    dx = rng.normal(0, 0.2, (n, 4)).astype(f32)
    ds = rng.normal(0, 1, (n, S)).astype(f32)
    mask = (rng.uniform(size=n) < 0.5).astype(f32)
    dt = f32(0.7)
    cfg2 = HashGridConfig.growing_2d()
    p2, s2 = O.euler_step(pos, st, dx, ds, 1, n, S, cfg2, float(dt), mask)
    m = mask[:, None]
    np.testing.assert_array_equal(p2[:, :2], pos[:, :2] + dt * dx[:, :2] * m)
    np.testing.assert_array_equal(p2[:, 2:], pos[:, 2:])
    np.testing.assert_array_equal(s2, st + dt * ds * m)
    cfg3 = HashGridConfig.growing_3dgs()
    p3, _ = O.euler_step(pos, st, dx, ds, 1, n, S, cfg3, float(dt), mask)
    np.testing.assert_array_equal(p3, pos + dt * dx * m)  # all four lanes in 3D
    tex = HashGridConfig.texture_2d()  # periodic, extent 2.0
    pw, _ = O.euler_step(np.array([[0.95, -0.95, 0, 0]], f32), np.zeros(1, f32),
                         np.array([[0.1, -0.1, 0, 0]], f32), np.zeros(1, f32), 1, 1, 1, tex, 1.0)
    assert pw[0, 0] == pytest.approx(-0.95, abs=1e-6) and pw[0, 1] == pytest.approx(0.95, abs=1e-6)


# --------------------------------------------------------------------------------------------
# step, rollout, mask
# --------------------------------------------------------------------------------------------

def _small_c1(n=512, seed=42, **model_kw):
    w = syn.workload("c1", seed=seed, particles=n)
    if model_kw:
        w["model"] = w["model"].replace(**model_kw)
        w["weights"] = syn.seeded_weights(w["model"], seed)
    return w


def test_step_is_perceive_then_mlp_then_euler():
    """NpaModel::step_cpu (model.rs:768-858): perceive with the model's options and hybrid
    gradient on, forward_from_features_with_eps(grid eps), euler_step with the mask."""
    w = _small_c1(400, density_grad=True)
    m, grid = w["model"], w["grid"]
    n = w["n"]
    mask = O.update_mask(1, n, 0.5, 3, 42)
    out = O.step(m, w["weights"], w["positions"], w["states"], 1, n, grid, 1.0, mask)
    per = O.perceive_with_options(w["positions"], w["states"], 1, n, m.state_dims, grid,
                                  m.perception_options())
    dx, ds = O.forward_from_features_with_eps(m, w["weights"], per.features, grid.eps)
    npos, nst = O.euler_step(w["positions"], w["states"], dx, ds, 1, n, m.state_dims, grid, 1.0,
                             mask)
    np.testing.assert_array_equal(out.next_positions, npos)
    np.testing.assert_array_equal(out.next_states, nst)
    np.testing.assert_array_equal(out.density, per.density)


def test_scale_equivariant_step_preserves_scaled_rollout():
    """scale_equivariant_cpu_step_preserves_scaled_rollout
    (crates/burn_automata/tests/core/equivariance.rs:4-67): 32 particles in a disk of radius
    0.2, hidden 8, ParticleDensityAndScale, scale 1.7 -> |base - scaled/scale| < 2e-4."""
    ka = KNOWN["scale_equivariant_cpu_step_preserves_scaled_rollout"]
    m = NpaConfig.growing_2d().replace(hidden_dims=ka["hidden_dims"],
                                       equivariance=EquivarianceMode.ParticleDensityAndScale)
    grid = HashGridConfig.growing_2d()
    weights = syn.seeded_weights(m, 17)
    n = ka["particles"]
    pos = syn.uniform_disk(n, seed=23, radius=ka["radius"])
    st = syn.normal_states(n, m.state_dims, seed=23, std=0.1)
    s = ka["scale"]
    spos = pos.copy()
    spos[:, :3] *= f32(s)
    base = O.step(m, weights, pos, st, 1, n, grid, 1.0)
    scaled = O.step(m, weights, spos, st, 1, n, grid.replace(eps=grid.eps * s), 1.0)
    tol = ka["tolerance"]
    assert np.max(np.abs(base.next_positions[:, :2] - scaled.next_positions[:, :2] / f32(s))) < tol
    assert np.max(np.abs(base.next_states - scaled.next_states)) < tol
    assert np.max(np.abs(base.next_positions[:, :2] - pos[:, :2])) > 1e-4  # it moved


def test_rollout_is_repeated_masked_steps():
    """run_rollout_from_particles (rollout/mod.rs:240-297) with the device mask schedule:
    step k uses update_mask(step index k)."""
    w = _small_c1(256)
    m, grid, n = w["model"], w["grid"], w["n"]
    pos, st = w["positions"].copy(), w["states"].copy()
    for k in range(4):
        mask = O.update_mask(1, n, 0.5, k, 42)
        out = O.step(m, w["weights"], pos, st, 1, n, grid, 1.0, mask)
        pos, st = out.next_positions, out.next_states
    rpos, rst = O.rollout(m, w["weights"], w["positions"], w["states"], 1, n, grid, 4, 1.0, 0.5, 42)
    np.testing.assert_array_equal(rpos, pos)
    np.testing.assert_array_equal(rst, st)


def test_mask_hash_matches_reference_cpu_replica():
    rng = np.random.default_rng(0)
    for v in list(rng.integers(0, 2 ** 32, 200)) + [0, 1, 61, M32]:
        assert O.hash_u32(int(v)) == hash_u32_ref(int(v))
    for p, s, seed in rng.integers(0, 2 ** 32, (100, 3)):
        assert O.random01(int(p), int(s), int(seed)) == random01_ref(int(p), int(s), int(seed))


def test_update_mask_lane_seeds_and_statistics():
    """gpu_update_mask (common.rs:115-124) with lane seeds gpu_random_seed(seed) ^ lane*N
    (crates/burn_automata/src/gpu/executor/state.rs:1282-1315)."""
    B, N, seed = 3, 1000, (7 << 32) | 42
    base = (seed & M32) ^ (seed >> 32)
    for step, p in [(0, 0.5), (5, 0.25)]:
        m = O.update_mask(B, N, p, step, seed)
        want = [float(random01_ref(i, step, base ^ (b * N)) < p) for b in range(B) for i in range(N)]
        np.testing.assert_array_equal(m, np.array(want, f32))
        assert abs(m.mean() - p) < 5 * math.sqrt(p * (1 - p) / m.size)
    assert np.all(O.update_mask(2, 64, 0.0, 1, 42) == 0)
    assert np.all(O.update_mask(2, 64, 1.0, 1, 42) == 1)


# --------------------------------------------------------------------------------------------
# decode
# --------------------------------------------------------------------------------------------

def test_gaussian_decode_known_answers():
    """splat_and_gaussian_decode_are_shape_stable (lib.rs:406-434) and
    gaussian_decode_modes_cover_fixed_learned_and_oriented_scale (lib.rs:437-482)."""
    ka = KNOWN["splat_and_gaussian_decode_are_shape_stable"]
    S = ka["state_dims"]
    st = np.zeros(S, f32)
    st[S - 3:] = ka["tail"]
    g = O.decode_gaussians_3d(np.zeros((1, 4), f32), st, S, GaussianDecodeConfig())
    assert g["spherical_harmonic"].shape == (1, 1, 3)
    np.testing.assert_array_equal(g["spherical_harmonic"][0, 0], np.array(ka["expect_sh"], f32))
    assert g["scale_opacity"][0, 3] > 0

    kb = KNOWN["gaussian_decode_modes_cover_fixed_learned_and_oriented_scale"]
    pos = np.array([kb["position"]], f32)
    learned = np.zeros(8, f32)
    for i, v in kb["learned_states"].items():
        learned[int(i)] = v
    g = O.decode_gaussians_3d(pos, learned, 8, GaussianDecodeConfig(
        mode=GaussianDecodeMode.GaussianSh0LearnedScale, sigma=0.01, opacity_scale=1.0))
    assert g["spherical_harmonic"].shape == (1, 1, 3)
    assert g["spherical_harmonic"][0, 0].tolist() == kb["expect_learned_sh"]
    assert g["scale_opacity"][0, 0] > 0.01 and g["scale_opacity"][0, 3] > 0.5
    assert g["rotation"][0].tolist() == [1.0, 0.0, 0.0, 0.0]
    oriented = np.zeros(20, f32)
    for i, v in kb["oriented_states"].items():
        oriented[int(i)] = v
    g = O.decode_gaussians_3d(pos, oriented, 20, GaussianDecodeConfig(
        mode=GaussianDecodeMode.GaussianSh0Oriented, sh_degree=1))
    assert g["spherical_harmonic"].shape == (1, 4, 3)
    assert abs(g["rotation"][0, 0] - 1.0) <= 1e-6
    assert np.isfinite(g["scale_opacity"][0, 0])


def test_fixed_decode_closed_form():
    """GaussianSh0FixedScale (gaussian.rs:53-223): colour clamp(tail + 0.5, 0, 1), scale
    clamp(sigma, min, max) on three axes, opacity clamp(opacity_scale, min, max), identity
    rotation, position passed through."""
    rng = np.random.default_rng(2)
    n, S = 40, 9
    pos = rng.uniform(-1, 1, (n, 4)).astype(f32)
    st = rng.normal(0, 0.6, (n, S)).astype(f32)
    cfg = GaussianDecodeConfig(sigma=0.5)
    g = O.decode_gaussians_3d(pos, st, S, cfg)
    np.testing.assert_array_equal(g["spherical_harmonic"][:, 0, :],
                                  np.clip(st[:, S - 3:] + f32(0.5), 0, 1))
    np.testing.assert_array_equal(g["position_visibility"][:, :3], pos[:, :3])
    assert np.all(g["scale_opacity"][:, :3] == f32(cfg.max_scale))
    assert np.all(g["scale_opacity"][:, 3] == f32(cfg.opacity_scale))
    assert np.all(g["rotation"] == np.array([1, 0, 0, 0], f32))


def test_learned_decode_closed_form():
    """GaussianSh0LearnedScale (gaussian.rs:172-184): scale = clamp(sigma exp(clamp(s[S-5], +-8)),
    min, max) on three axes; opacity = clamp(clamp(sigmoid(clamp(s[S-4], +-12)), min, max) *
    opacity_scale, min, max)."""
    from scipy.special import expit
    rng = np.random.default_rng(4)
    n, S = 300, 10
    st = rng.normal(0, 3, (n, S)).astype(f32)
    cfg = GaussianDecodeConfig(mode=GaussianDecodeMode.GaussianSh0LearnedScale, sigma=0.02,
                               min_scale=0.005, max_scale=0.2, opacity_scale=0.8)
    g = O.decode_gaussians_3d(np.zeros((n, 4), f32), st, S, cfg)
    sc = np.clip(0.02 * np.exp(np.clip(st[:, S - 5].astype(np.float64), -8, 8)), 0.005, 0.2)
    op = np.clip(np.clip(expit(np.clip(st[:, S - 4].astype(np.float64), -12, 12)), 0.001, 0.95) * 0.8,
                 0.001, 0.95)
    for k in range(3):
        np.testing.assert_allclose(g["scale_opacity"][:, k], sc, rtol=2e-6)
    np.testing.assert_allclose(g["scale_opacity"][:, 3], op, rtol=2e-6)
    assert ((sc > 0.005) & (sc < 0.2)).sum() > n // 4


# --------------------------------------------------------------------------------------------
# viewer export (write_gaussian_from_output, gpu_step.wgsl:4963-5052)
# --------------------------------------------------------------------------------------------

def _quat_rotate(q, v):
    """Rotates v by the unit quaternion q = (w, x, y, z), in float64."""
    w, x, y, z = (np.asarray(q, np.float64)[..., k] for k in range(4))
    R = np.stack([np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
                  np.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
                  np.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1)], -2)
    return np.einsum("...ij,...j->...i", R, np.asarray(v, np.float64))


def test_export_buffer_contents_known_properties():
    """wgpu_state_writes_gaussian_buffers_on_gpu (tests/gpu_wgpu/gaussian.rs:243-310) on a growing-3DGS
    model: positions copied, visibility 1, identity rotation (no position features), finite positive
    scale max(eps * 0.12, 8e-5), opacity clamp(sigmoid(channel 8), 0.001, 0.95); the 48 SH floats are
    zero but for the DC triple, which decodes back (SH_C0 * dc + 0.5) to clamp(tail + 0.5, 0, 1) of
    channels S-3, S-2, S-1 in that order."""
    from scipy.special import expit
    rng = np.random.default_rng(11)
    m, g = NpaConfig.growing_3dgs(), HashGridConfig.growing_3dgs()
    n, S = 64, m.state_dims
    pos = rng.uniform(-1, 1, (n, 4)).astype(f32)
    st = rng.normal(0, 1.5, (n, S)).astype(f32)
    ex = O.write_gaussians(pos, st, n, m, g)
    np.testing.assert_array_equal(ex["position_visibility"][:, :3], pos[:, :3])
    assert np.all(ex["position_visibility"][:, 3] == 1.0)
    assert np.all(ex["rotation"] == np.array([1, 0, 0, 0], f32))
    assert np.all(ex["scale_opacity"][:, :3] == f32(max(f32(g.eps) * f32(0.12), f32(0.00008))))
    np.testing.assert_allclose(ex["scale_opacity"][:, 3], np.clip(expit(st[:, 8].astype(np.float64)), 0.001, 0.95),
                               rtol=1e-6)
    sh = ex["spherical_harmonic"]
    assert sh.shape == (n, 48) and not sh[:, 3:].any()
    colour = np.clip(st[:, S - 3:].astype(np.float64) + 0.5, 0, 1)
    np.testing.assert_allclose(sh[:, :3] * 0.28209479177387814 + 0.5, colour, atol=1e-6)
    assert np.unique(np.round(colour, 3)).size > 20  # distinct tail channels: their order is pinned


def test_export_2d_and_small_state_rules():
    """2D: z written as 0, opacity 1, scale floor 8e-5 at tiny eps. Fewer than three state channels:
    the missing tail channels read channel 0 (output_tail_state_channel gpu_step.wgsl:1577-1583). A 3D
    state of at most 8 channels takes the opacity logit from channel 3 (1585-1591)."""
    from scipy.special import expit
    rng = np.random.default_rng(12)
    n = 20
    pos = rng.uniform(-1, 1, (n, 4)).astype(f32)
    m2 = NpaConfig.growing_2d().replace(state_dims=5)
    st = rng.normal(0, 1, (n, 5)).astype(f32)
    for eps, want_scale in ((0.05, max(f32(0.05) * f32(0.12), f32(0.00008))), (1e-4, f32(0.00008))):
        ex = O.write_gaussians(pos, st, n, m2, HashGridConfig.growing_2d().replace(eps=eps))
        assert np.all(ex["position_visibility"][:, 2] == 0.0)
        np.testing.assert_array_equal(ex["position_visibility"][:, :2], pos[:, :2])
        assert np.all(ex["scale_opacity"][:, 3] == 1.0)
        assert np.all(ex["scale_opacity"][:, :3] == f32(want_scale))
    m1 = NpaConfig.growing_2d().replace(state_dims=1)
    ex = O.write_gaussians(pos, st[:, :1], n, m1, HashGridConfig.growing_2d())
    dc = ex["spherical_harmonic"][:, :3] * 0.28209479177387814 + 0.5
    np.testing.assert_allclose(dc, np.repeat(np.clip(st[:, :1] + 0.5, 0, 1), 3, axis=1), atol=1e-6)
    m3 = NpaConfig.growing_3dgs().replace(state_dims=8)
    ex = O.write_gaussians(pos, st[:, :5].repeat(2, axis=1)[:, :8], n, m3, HashGridConfig.growing_3dgs())
    logit = st[:, :5].repeat(2, axis=1)[:, 3].astype(np.float64)
    np.testing.assert_allclose(ex["scale_opacity"][:, 3], np.clip(expit(logit), 0.001, 0.95), rtol=1e-6)


def test_export_surface_normal_branch():
    """3D models with position features and S >= 9 (gpu_step.wgsl:5000-5040): the quaternion takes +z
    onto the unit normal of channels 4..6 (normal near -z: the half turn (0, 1, 0, 0); degenerate
    normal: +z, identity); tangent t = max(clamp(0.32 eps clamp(sqrt(4096 / N), 0.4, 2), 0.08 eps,
    0.64 eps), 8e-5) on x and y, max(0.18 t, 8e-5) on z. S = 8 keeps the isotropic branch."""
    rng = np.random.default_rng(13)
    m = NpaConfig.torus_field_3dgs().replace(state_dims=12)
    g = HashGridConfig.growing_3dgs()
    n = 200
    pos = rng.uniform(-1, 1, (n, 4)).astype(f32)
    st = rng.normal(0, 1, (n, 12)).astype(f32)
    st[0, 4:7] = (0.0, 0.0, 0.0)          # degenerate: identity
    st[1, 4:7] = (1e-4, -2e-4, -3.0)      # within 1e-6 of -z: half turn about x
    st[2, 4:7] = (0.0, 0.0, 2.5)          # +z: identity
    for N, scale in ((100, 2.0), (4096, 1.0), (16384, 0.5), (65536, 0.4)):
        ex = O.write_gaussians(pos, st, N, m, g)
        q = ex["rotation"].astype(np.float64)
        np.testing.assert_allclose(np.linalg.norm(q, axis=1), 1.0, atol=1e-6)
        nrm = st[3:, 4:7].astype(np.float64)
        unit = nrm / np.linalg.norm(nrm, axis=1, keepdims=True)
        np.testing.assert_allclose(_quat_rotate(q[3:], [0, 0, 1]), unit, atol=2e-6)
        np.testing.assert_array_equal(ex["rotation"][0], np.array([1, 0, 0, 0], f32))
        np.testing.assert_array_equal(ex["rotation"][1], np.array([0, 1, 0, 0], f32))
        np.testing.assert_array_equal(ex["rotation"][2], np.array([1, 0, 0, 0], f32))
        eps = float(np.float32(g.eps))
        t = max(min(max(0.32 * eps * scale, 0.08 * eps), 0.64 * eps), 8e-5)
        np.testing.assert_allclose(ex["scale_opacity"][:, 0], t, rtol=1e-6)
        np.testing.assert_allclose(ex["scale_opacity"][:, 1], t, rtol=1e-6)
        np.testing.assert_allclose(ex["scale_opacity"][:, 2], max(0.18 * t, 8e-5), rtol=1e-6)
    ex8 = O.write_gaussians(pos, st[:, :8], 4096, m.replace(state_dims=8), g)
    assert np.all(ex8["rotation"] == np.array([1, 0, 0, 0], f32))
    assert np.all(ex8["scale_opacity"][:, :3] == f32(max(f32(g.eps) * f32(0.12), f32(0.00008))))


# --------------------------------------------------------------------------------------------
# splat
# --------------------------------------------------------------------------------------------

def test_splat_shape_known_answer():
    """splat_and_gaussian_decode_are_shape_stable (lib.rs:406-418)."""
    img = O.splat_particles_2d(np.zeros((1, 4), f32), np.array([[1, 0, 0]], f32),
                               Splat2dConfig(image_size=8))
    assert img.shape == (64, 4) and np.any(img[:, 3] > 0)


@pytest.mark.parametrize("y_up", [True, False])
def test_single_particle_splat_is_a_normalised_gaussian(y_up):
    """splat_particles_2d (splat.rs:30-93): one particle -> exp(-r^2/2s^2) over the
    (2 ceil(5s)+1)^2 footprint, normalised to norm_scale, colour times alpha."""
    size, sigma_w = 64, 2.3  # sigma in pixels of a (hi - lo) / size grid
    cfg = Splat2dConfig(image_size=size, sigma=sigma_w, y_up=y_up, pixel_size=2.0 / size)
    p = np.array([[0.131, -0.377, 0, 0]], f32)
    c = np.array([[0.2, 0.7, 1.0]], f32)
    img = O.splat_particles_2d(p, c, cfg).reshape(size, size, 4).astype(np.float64)
    sig = sigma_w * size * cfg.pixel_size / (cfg.hi - cfg.lo)
    rad = max(math.ceil(5 * sig), 1)
    px = (0.131 + 1) / 2 * (size - 1)
    py = (-0.377 + 1) / 2 * (size - 1)
    if y_up:
        py = (size - 1) - py
    bx, by = math.floor(px), math.floor(py)
    want = np.zeros((size, size))
    for oy in range(-rad, rad + 1):
        for ox in range(-rad, rad + 1):
            dx, dy = ox - (px - bx), oy - (py - by)
            want[by + oy, bx + ox] = math.exp(-(dx * dx + dy * dy) / (2 * sig * sig))
    norm = (size * cfg.pixel_size / (cfg.hi - cfg.lo)) ** 2
    want = want / want.sum() * norm
    assert rel(img[:, :, 3], want) < 2e-5
    for ch in range(3):
        assert rel(img[:, :, ch], want * float(c[0, ch])) < 2e-5
    assert img[:, :, 3].sum() == pytest.approx(norm, rel=1e-5)


def test_splat_is_additive_and_clips_at_the_border():
    rng = np.random.default_rng(6)
    n = 300
    pos = np.zeros((n, 4), f32)
    pos[:, :2] = rng.uniform(-1.05, 1.05, (n, 2))
    col = rng.uniform(0, 1, (n, 3)).astype(f32)
    cfg = Splat2dConfig(image_size=48, sigma=1.4, pixel_size=2.0 / 48)
    a = O.splat_particles_2d(pos[:150], col[:150], cfg).astype(np.float64)
    b = O.splat_particles_2d(pos[150:], col[150:], cfg).astype(np.float64)
    ab = O.splat_particles_2d(pos, col, cfg)
    assert rel(ab, a + b) < 1e-6
    # a particle outside the image keeps only its in-bounds weights, still normalised to 1
    one = O.splat_particles_2d(np.array([[0.99, 0.99, 0, 0]], f32), np.ones((1, 3), f32), cfg)
    norm = (48 * cfg.pixel_size / 2.0) ** 2
    assert one[:, 3].sum() == pytest.approx(norm, rel=1e-5)


@pytest.mark.parametrize("name,particles", [("c1", 2048), ("c4", 4096), ("c3", 8192),
                                            ("torus", 1024)])
def test_sampled_rows_equal_the_full_pass(name, particles):
    """density_rows / step_rows (the sampled evaluation used at C3's full size) give exactly the
    rows of the full density pass and the full step, incl. 3D gates and masked-out particles."""
    if name == "torus":
        m, g = NpaConfig.torus_field_3dgs(), HashGridConfig.growing_3dgs()
        pos = syn.uniform_ball(particles, 6, 0.5)
        pos[::7, 3] = 1.0
        st = syn.normal_states(particles, m.state_dims, 6, std=1.0)
        st[:, 3] += 3.5
        w = {"model": m, "grid": g, "batch": 1, "n": particles, "positions": pos, "states": st,
             "weights": syn.seeded_weights(m, 6)}
    else:
        w = syn.workload(name, particles=particles)
    b, n = w["batch"], w["n"]
    mask = O.update_mask(b, n, 0.5, 3, 42)
    full = O.step(w["model"], w["weights"], w["positions"], w["states"], b, n, w["grid"], 1.0,
                  mask)
    sel = np.random.default_rng(1).choice(b * n, 300, replace=False).astype(np.uint32)
    np.testing.assert_array_equal(O.density_rows(w["positions"], b, n, w["grid"], sel),
                                  full.density[sel])
    p, s = O.step_rows(w["model"], w["weights"], w["positions"], w["states"], b, n, w["grid"],
                       1.0, mask, full.density, sel)
    np.testing.assert_array_equal(p, full.next_positions[sel])
    np.testing.assert_array_equal(s, full.next_states[sel])


# ------------------------------------------------------------------ 3D render raster
def _moments(img, size):
    """Total alpha, alpha-weighted centroid (column, row) and per-axis variance of one image."""
    a = img[:, 3].astype(np.float64).reshape(size, size)
    ys, xs = np.mgrid[0:size, 0:size]
    tot = a.sum()
    cx, cy = (a * xs).sum() / tot, (a * ys).sum() / tot
    vx, vy = (a * (xs - cx) ** 2).sum() / tot, (a * (ys - cy) ** 2).sum() / tot
    return tot, cx, cy, vx, vy


def test_view_bases_are_right_handed_orthonormal_frames():
    """view_basis (render_loss/projection.rs:31-43): the axis views pick coordinate axes; the
    iso view looks along (right x up) with right = (1,-1,0)/sqrt2 and up = (1,1,2)/sqrt6."""
    from burn_automata_amd.config import RenderViewPreset as V
    e = np.eye(3, dtype=f32)
    for v, (r, u, fw) in {V.Xy: (0, 1, 2), V.Xz: (0, 2, 1), V.Yz: (1, 2, 0)}.items():
        got = O.view_basis(v)
        for g, k in zip(got, (r, u, fw)):
            np.testing.assert_array_equal(g, e[k])
    r, u, fw = (b.astype(np.float64) for b in O.view_basis(V.Iso))
    np.testing.assert_allclose(r, np.array([1, -1, 0]) / math.sqrt(2), rtol=0, atol=1e-7)
    np.testing.assert_allclose(u, np.array([1, 1, 2]) / math.sqrt(6), rtol=0, atol=1e-7)
    np.testing.assert_allclose(fw, np.array([-1, -1, 1]) / math.sqrt(3), rtol=0, atol=1e-7)
    m = np.stack([r, u, fw])
    np.testing.assert_allclose(m @ m.T, np.eye(3), atol=1e-6)
    assert np.linalg.det(m) == pytest.approx(1.0, abs=1e-6)


def test_project_positions_is_a_rotation_with_clamped_depth():
    """project_positions (projection.rs:11-29): (x, y) = coordinates along right and up; depth
    = clamp(0.5 + 0.5 forward.p / world_scale, 0, 1); the position's w is ignored."""
    from burn_automata_amd.config import ALL_VIEWS
    rng = np.random.default_rng(11)
    pos = rng.uniform(-2, 2, (500, 4)).astype(f32)
    ws = 1.25
    for v in ALL_VIEWS:
        r, u, fw = (b.astype(np.float64) for b in O.view_basis(v))
        pp = O.project_positions(v, pos, ws).astype(np.float64)
        p3 = pos[:, :3].astype(np.float64)
        np.testing.assert_allclose(pp[:, 0], p3 @ r, atol=2e-6)
        np.testing.assert_allclose(pp[:, 1], p3 @ u, atol=2e-6)
        np.testing.assert_allclose(pp[:, 2], np.clip(0.5 + 0.5 * (p3 @ fw) / ws, 0, 1), atol=2e-6)
        # a rotation keeps lengths: x^2 + y^2 + (forward.p)^2 = |p|^2
        np.testing.assert_allclose(pp[:, 0] ** 2 + pp[:, 1] ** 2 + (p3 @ fw) ** 2,
                                   (p3 ** 2).sum(1), rtol=1e-5)
    pos2 = pos.copy()
    pos2[:, 3] = 123.0
    np.testing.assert_array_equal(O.project_positions(3, pos2, ws), O.project_positions(3, pos, ws))


@pytest.mark.parametrize("sigma", [0.9, 2.5, 4.2])
def test_projected_splat_of_one_particle_has_the_gaussian_moments(sigma):
    """splat_projected (render_loss/image.rs:18-79) of one particle well inside the image: total
    alpha = opacity, colour and depth_sum = colour and depth times alpha, centroid = the projected
    pixel ((x+ws)/2ws (size-1), (ws-y)/2ws (size-1)), per-axis variance sigma^2, support radius
    ceil(5 sigma)."""
    from burn_automata_amd.config import RenderLossConfig
    size, ws = 64, 1.25
    cfg = RenderLossConfig(image_size=size, world_scale=ws)
    x, y, depth, op = 0.213, -0.161, 0.37, 0.64
    col = np.array([[0.2, 0.7, 1.0]], f32)
    img = O.splat_projected(np.array([[x, y, depth]], f32), col, np.array([op], f32),
                            np.array([sigma], f32), cfg)
    tot, cx, cy, vx, vy = _moments(img, size)
    assert tot == pytest.approx(op, rel=1e-5)
    np.testing.assert_allclose(img[:, :3].sum(0), col[0] * op, rtol=1e-5)
    assert img[:, 4].sum() == pytest.approx(depth * op, rel=1e-5)
    assert cx == pytest.approx((x + ws) / (2 * ws) * (size - 1), abs=1e-3)
    assert cy == pytest.approx((ws - y) / (2 * ws) * (size - 1), abs=1e-3)
    assert vx == pytest.approx(sigma ** 2, rel=2e-3) and vy == pytest.approx(sigma ** 2, rel=2e-3)
    a = img[:, 3].reshape(size, size)
    cols = np.nonzero(a.any(0))[0]
    bx = math.floor((x + ws) / (2 * ws) * (size - 1))
    rad = math.ceil(5 * sigma)
    assert cols.min() == bx - rad and cols.max() == bx + rad


def test_projected_splat_clamps_sigma_and_opacity_and_divides_by_count():
    """sigma is clamped to [min_sigma, max_sigma], opacity to [0, 1]; every particle's weights
    carry 1/count (image.rs:29, 39, 69-71); edge particles renormalise over in-bounds pixels."""
    from burn_automata_amd.config import RenderLossConfig
    size = 64
    cfg = RenderLossConfig(image_size=size, min_sigma=1.5, max_sigma=3.0)
    pp = np.array([[0.0, 0.0, 0.5]], f32)
    col = np.ones((1, 3), f32)
    for s, want in ((0.2, 1.5), (2.0, 2.0), (9.0, 3.0)):
        _, _, _, vx, _ = _moments(O.splat_projected(pp, col, np.ones(1, f32), np.array([s], f32), cfg), size)
        assert vx == pytest.approx(want ** 2, rel=2e-3), s
    assert O.splat_projected(pp, col, np.array([1.7], f32), np.array([2.0], f32), cfg)[:, 3].sum() == \
        pytest.approx(1.0, rel=1e-5)
    assert not O.splat_projected(pp, col, np.array([-0.3], f32), np.array([2.0], f32), cfg).any()
    # two copies of one particle draw the single particle's image (each at weight 1/2)
    one = O.splat_projected(pp, col, np.ones(1, f32), np.array([2.0], f32), cfg)
    two = O.splat_projected(np.repeat(pp, 2, 0), np.repeat(col, 2, 0), np.ones(2, f32),
                            np.full(2, 2.0, f32), cfg)
    assert rel(two, one) < 1e-6
    # a particle at the image corner keeps its full alpha on the pixels that remain
    corner = O.splat_projected(np.array([[1.25, 1.25, 0.5]], f32), col, np.ones(1, f32),
                               np.array([2.5], f32), cfg)
    assert corner[:, 3].sum() == pytest.approx(1.0, rel=1e-5)
    assert corner[:, 3].reshape(size, size)[0, size - 1] == corner[:, 3].max()
    far = O.splat_projected(np.array([[9.0, 0.0, 0.5]], f32), col, np.ones(1, f32), np.array([2.5], f32), cfg)
    assert not far.any()


def test_projected_splat_is_linear_in_the_particle_sets():
    from burn_automata_amd.config import RenderLossConfig
    rng = np.random.default_rng(12)
    n = 400
    pp = np.concatenate([rng.uniform(-1.4, 1.4, (n, 2)), rng.uniform(0, 1, (n, 1))], 1).astype(f32)
    col, op = rng.uniform(0, 1, (n, 3)).astype(f32), rng.uniform(0, 1, n).astype(f32)
    sg = rng.uniform(0.5, 6, n).astype(f32)
    cfg = RenderLossConfig(image_size=48)
    a = O.splat_projected(pp[:100], col[:100], op[:100], sg[:100], cfg).astype(np.float64)
    b = O.splat_projected(pp[100:], col[100:], op[100:], sg[100:], cfg).astype(np.float64)
    ab = O.splat_projected(pp, col, op, sg, cfg)
    assert rel(ab, (100 * a + 300 * b) / 400) < 1e-5


def test_render_attributes_follow_the_state_tail():
    """state_tail_render_attributes (render_loss/attributes.rs:15-87): colour = clamp(tail+0.5),
    opacity = clamp(sigmoid(state[8 if S > 8 else 3] + bias), 0.001, 0.95) (0.95 when S <= 3;
    rollout/mod.rs:37-45), sigma by decode mode, learned logit from state[S-5] clamped to +-8."""
    from scipy.special import expit
    from burn_automata_amd.config import RenderLossConfig
    rng = np.random.default_rng(13)
    n = 300
    for S, ch in ((16, 8), (9, 8), (8, 3), (5, 3), (4, 3), (3, None)):
        st = rng.normal(0, 3, (n, S)).astype(f32)
        cfg = RenderLossConfig(opacity_logit_bias=0.7)
        col, op, sg, dv = O.render_attributes(st, S, cfg)
        np.testing.assert_array_equal(col, np.clip(st[:, S - 3:] + f32(0.5), 0, 1))
        if ch is None:
            np.testing.assert_array_equal(op, np.full(n, 0.95, f32))
        else:
            want = np.clip(expit(st[:, ch].astype(np.float64) + np.float64(f32(0.7))), 0.001, 0.95)
            np.testing.assert_allclose(op, want, rtol=2e-6)
            other = st.copy()
            other[:, [c for c in range(S) if c != ch]] = 0
            np.testing.assert_array_equal(O.render_attributes(other, S, cfg)[1], op)
        np.testing.assert_array_equal(sg, np.full(n, 2.5, f32))
        assert not dv.any()
    S = 16
    st = rng.normal(0, 4, (n, S)).astype(f32)
    cfg = RenderLossConfig(gaussian_decode_mode=GaussianDecodeMode.GaussianSh0LearnedScale, sigma=2.0,
                           min_sigma=0.5, max_sigma=6.0)
    _, _, sg, dv = O.render_attributes(st, S, cfg)
    raw = 2.0 * np.exp(np.clip(st[:, S - 5].astype(np.float64), -8, 8))
    np.testing.assert_allclose(sg, np.clip(raw, 0.5, 6.0), rtol=2e-6)
    inside = (raw > 0.5) & (raw < 6.0)
    np.testing.assert_allclose(dv[inside], raw[inside], rtol=2e-6)
    assert not dv[~inside].any() and inside.any() and (~inside).any()
    _, _, sg, _ = O.render_attributes(st, S, cfg.replace(gaussian_decode_mode=GaussianDecodeMode.ParticlePoint))
    np.testing.assert_array_equal(sg, np.full(n, 0.5, f32))
    _, _, sg, _ = O.render_attributes(st, S, cfg.replace(gaussian_decode_mode=GaussianDecodeMode.GaussianSh0Oriented,
                                                          sigma=9.0))
    np.testing.assert_array_equal(sg, np.full(n, 6.0, f32))
    from burn_automata_amd import _abi
    with pytest.raises(_abi.InvalidArgument):
        O.render_attributes(np.zeros((4, 2), f32), 2, RenderLossConfig())
    with pytest.raises(_abi.InvalidArgument):
        O.render_attributes(np.zeros((4, 4), f32), 4, cfg)


def test_render_defaults_match_the_reference():
    """RenderLossConfig::default (render_loss.rs:48-63) and the opacity limits (render_loss.rs:21-23)."""
    from burn_automata_amd.config import RenderLossConfig
    c = RenderLossConfig()
    assert (c.image_size, c.sigma, c.min_sigma, c.max_sigma, c.world_scale, c.target_samples) == \
        (64, 2.5, 0.75, 5.0, 1.25, 8192)
    assert c.gaussian_decode_mode == GaussianDecodeMode.GaussianSh0FixedScale
    st = np.zeros((2, 16), f32)
    st[0, 8], st[1, 8] = 40.0, -40.0
    _, op, _, _ = O.render_attributes(st, 16, c)
    np.testing.assert_array_equal(op, np.array([0.95, 0.001], f32))


# ------------------------------------------------------------------ perception adjoint
def _adjoint_fixture(eps):
    cfg = HashGridConfig(3, Boundary.Clamped, HashGridMode.Particle, (8, 8, 8), eps, 16)
    states = np.array([0.10, -0.20, 0.05, 0.30, 0.15, -0.10, -0.25, 0.35, 0.20, 0.05, -0.30, 0.40], f32)
    return cfg, states


def _adj_opts(cfg, hybrid, position_features):
    return PerceptionOptions(state_grad=True, density_grad=True, eps0=cfg.eps, scale_equivariance=True,
                             particle_density_equivariance=True, log_norm_grad=True,
                             log_norm_density_grad=True, hybrid_state_gradient=hybrid,
                             position_features=position_features)


def _loss(pos, st, n, S, cfg, opts, fa):
    """sum(features * feature_adjoint), the scalar the reference's finite differences use."""
    f = O.perceive_with_options(pos, st, 1, n, S, cfg, opts).features.astype(np.float64)
    return float((f.ravel() * fa.astype(np.float64)).sum())


def test_adjoint_reference_state_finite_difference():
    """perceive_state_adjoint_matches_finite_difference (lib.rs:123-198), its fixture and bound."""
    cfg, st = _adjoint_fixture(0.35)
    pos = np.array([[0, 0, 0, 0], [0.12, 0.04, -0.03, 0], [-0.08, 0.10, 0.02, 0], [0.04, -0.09, 0.11, 0]], f32)
    opts = _adj_opts(cfg, True, False)
    F = opts.feature_dims(3, 3)
    fa = (np.sin((np.arange(4 * F, dtype=f32) + f32(1)) * f32(0.017)) * f32(0.1)).astype(f32)
    adj = O.perceive_state_adjoint_with_options(pos, st, 1, 4, 3, cfg, opts, fa)
    e = 1e-3
    p, m = st.copy(), st.copy()
    p[4] += f32(e)
    m[4] -= f32(e)
    fd = (_loss(pos, p, 4, 3, cfg, opts, fa) - _loss(pos, m, 4, 3, cfg, opts, fa)) / (2 * e)
    assert abs(adj[4] - fd) <= 2e-3, (adj[4], fd)


@pytest.mark.parametrize("hybrid,particle,axis,tol,phase,amp,shift", [
    (False, 1, 0, 7.5e-2, 0.013, 0.05, 3.0),   # lib.rs:201-277
    (True, 2, 1, 2.5e-1, 0.011, 0.03, 5.0),    # lib.rs:280-356
])
def test_adjoint_reference_position_finite_difference(hybrid, particle, axis, tol, phase, amp, shift):
    """perceive_position_adjoint_matches_finite_difference_{without,with}_hybrid_moment."""
    cfg, st = _adjoint_fixture(0.40)
    pos = np.array([[0, 0, 0, 0], [0.11, 0.03, -0.02, 0], [-0.07, 0.09, 0.04, 0], [0.05, -0.08, 0.10, 0]], f32)
    opts = _adj_opts(cfg, hybrid, True)
    F = opts.feature_dims(3, 3)
    k = np.arange(4 * F, dtype=f32) + f32(shift)
    fa = ((np.sin(k * f32(phase)) if hybrid else np.cos(k * f32(phase))) * f32(amp)).astype(f32)
    adj = O.perceive_adjoint_with_options(pos, st, 1, 4, 3, cfg, opts, fa)
    e = 1e-4
    p, m = pos.copy(), pos.copy()
    p[particle, axis] += f32(e)
    m[particle, axis] -= f32(e)
    fd = (_loss(p, st, 4, 3, cfg, opts, fa) - _loss(m, st, 4, 3, cfg, opts, fa)) / (2 * e)
    assert abs(adj.position[particle, axis] - fd) <= tol, (adj.position[particle, axis], fd)


ADJOINT_CASES = {
    # name: (dim, boundary, hybrid, state_grad, density_grad, log_norm, position_features)
    "2d_growing": (2, Boundary.Clamped, False, True, False, True, False),
    "2d_hybrid_dgrad": (2, Boundary.Clamped, True, True, True, True, True),
    "2d_periodic_plain": (2, Boundary.Periodic, False, True, True, False, False),
    "3d_hybrid": (3, Boundary.Clamped, True, True, True, True, True),
    "3d_blur_only": (3, Boundary.Clamped, False, False, False, False, True),
}


def _adjoint_case(name, n=14, S=3, seed=0):
    dim, bnd, hyb, sg, dg, ln, pf = ADJOINT_CASES[name]
    eps = 0.5
    gs = (4, 4, 4 if dim == 3 else 1)
    cfg = HashGridConfig(dim, bnd, HashGridMode.Grid, gs, eps, 16)
    rng = np.random.default_rng(seed)
    pos = np.zeros((n, 4), f32)
    lo = 0.55 if bnd == Boundary.Periodic else 0.05
    pos[:, :dim] = rng.uniform(lo, lo + 0.45, (n, dim))  # dense: every moment matrix well conditioned
    st = rng.normal(0, 0.5, n * S).astype(f32)
    opts = PerceptionOptions(state_grad=sg, density_grad=dg, eps0=0.35, scale_equivariance=True,
                             particle_density_equivariance=True, log_norm_grad=ln,
                             log_norm_density_grad=ln, hybrid_state_gradient=hyb, position_features=pf)
    F = opts.feature_dims(S, dim)
    fa = rng.normal(0, 0.1, n * F).astype(f32)
    return cfg, pos, st, opts, fa, n, S, dim


@pytest.mark.parametrize("name", sorted(ADJOINT_CASES))
def test_adjoint_is_the_gradient_of_the_forward(name):
    """Every state and position coordinate against central differences of the oracle's forward
    (states: step 3e-3; positions: 1e-3; f32 forward, float64 loss).
    A dropped or mis-signed term of adjoint.rs shows up as an O(1) relative error."""
    cfg, pos, st, opts, fa, n, S, dim = _adjoint_case(name)
    adj = O.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, fa)
    fd_s = np.zeros(n * S)
    for k in range(n * S):
        p, m = st.copy(), st.copy()
        p[k] += f32(3e-3)
        m[k] -= f32(3e-3)
        fd_s[k] = (_loss(pos, p, n, S, cfg, opts, fa) - _loss(pos, m, n, S, cfg, opts, fa)) / (
            float(p[k]) - float(m[k]))
    fd_p = np.zeros((n, dim))
    for i in range(n):
        for a in range(dim):
            p, m = pos.copy(), pos.copy()
            p[i, a] += f32(1e-3)
            m[i, a] -= f32(1e-3)
            fd_p[i, a] = (_loss(p, st, n, S, cfg, opts, fa) - _loss(m, st, n, S, cfg, opts, fa)) / (
                float(p[i, a]) - float(m[i, a]))
    es = np.abs(adj.state - fd_s).max() / np.abs(fd_s).max()
    ep = np.abs(adj.position[:, :dim] - fd_p).max() / np.abs(fd_p).max()
    assert es < 1e-3 and ep < 1e-2, (es, ep)
    assert not adj.position[:, dim:].any()


def test_adjoint_is_linear_and_carries_identity_rows():
    cfg, pos, st, opts, fa, n, S, dim = _adjoint_case("2d_hybrid_dgrad")
    F = opts.feature_dims(S, dim)
    rng = np.random.default_rng(9)
    fb = rng.normal(0, 0.1, n * F).astype(f32)
    a = O.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, fa)
    b = O.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, fb)
    ab = O.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, fa + fb)
    assert rel(ab.state, a.state.astype(np.float64) + b.state) < 1e-5
    assert rel(ab.position, a.position.astype(np.float64) + b.position) < 1e-5
    # only the identity rows set: state adjoint == those rows; only the position rows: position
    only = np.zeros((n, F), f32)
    only[:, :S] = fa.reshape(n, F)[:, :S]
    r = O.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, only)
    np.testing.assert_array_equal(r.state, only[:, :S].ravel())
    assert not r.position.any()
    only = np.zeros((n, F), f32)
    only[:, F - dim:] = fa.reshape(n, F)[:, F - dim:]
    r = O.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, only)
    np.testing.assert_array_equal(r.position[:, :dim], only[:, F - dim:])
    assert not r.state.any()


# ---------------------------------------------------------------- oriented Gaussian raster
# The reference's viewer draws the planar export through the un-vendored bevy_gaussian_splatting
# 8.0.1; no reference test pins its pixels. The oracle's restatement of the published 3D Gaussian
# splatting forward pass is pinned here by closed forms computed independently in float64.
from burn_automata_amd.config import RasterCamera, RasterColor  # noqa: E402


def _raster_one(cam, pos, scale, quat=(1.0, 0.0, 0.0, 0.0), opacity=0.8, sh=(0.3, 0.1, -0.2)):
    pv = np.array([[*pos, 1.0]], f32)
    so = np.array([[*scale, opacity]], f32)
    return O.raster_gaussians_3d(pv, np.array(sh, f32), np.array([quat], f32), so, cam)


def _expected_alpha(cam, a, b, c, mx, my, opacity):
    """alpha over the image of one Gaussian with 2D covariance [[a, b], [b, c]] (0.3 included)
    centred at (mx, my): min(0.99, o e^power), zero below 1/255 or outside its 3-sigma tiles."""
    det = a * c - b * b
    ca, cb, cc = c / det, -b / det, a / det
    ys, xs = np.mgrid[0:cam.height, 0:cam.width].astype(np.float64)
    dx, dy = mx - (xs + 0.5), my - (ys + 0.5)
    power = -0.5 * (ca * dx * dx + cc * dy * dy) - cb * dx * dy
    alpha = np.minimum(0.99, opacity * np.exp(power))
    alpha[(power > 0) | (alpha < 1 / 255)] = 0.0
    mid = 0.5 * (a + c)
    r = math.ceil(3 * math.sqrt(mid + math.sqrt(max(0.1, mid * mid - det))))
    tx, ty = xs // 16, ys // 16
    inside = ((tx >= max(0, math.floor((mx - r) / 16))) & (tx < math.floor((mx + r) / 16) + 1) &
              (ty >= max(0, math.floor((my - r) / 16))) & (ty < math.floor((my + r) / 16) + 1))
    return np.where(inside, alpha, 0.0)


@pytest.mark.parametrize("opacity", [0.8, 1.0])
def test_raster_centred_isotropic_closed_form(opacity):
    """A sphere of radius s on the optical axis at distance z: Sigma2d = (f s / z)^2 I + 0.3 I, so
    every pixel is colour * alpha(d^2) with the centre clamped at 0.99 when the opacity is 1."""
    cam = RasterCamera.look_at((0, 0, 3), width=64, height=48, color_mode=RasterColor.Rgb)
    s = 0.1 if opacity < 1 else 0.3  # wide enough that the centre pixels reach the 0.99 clamp
    img = _raster_one(cam, (0, 0, 0), (s, s, s), opacity=opacity, sh=(0.9, 0.5, 0.25))
    var = (cam.fx * s / 3.0) ** 2 + 0.3
    alpha = _expected_alpha(cam, var, 0.0, var, cam.cx, cam.cy, opacity)
    np.testing.assert_allclose(img[..., 3], alpha, atol=2e-6)
    for ch, col in enumerate((0.9, 0.5, 0.25)):
        np.testing.assert_allclose(img[..., ch], col * alpha, atol=2e-6)
    if opacity == 1.0:
        assert img[..., 3].max() == np.float32(0.99) and (img[..., 3] == np.float32(0.99)).sum() >= 4


def test_raster_off_axis_centre_and_y_flip():
    """The alpha centroid of a small Gaussian sits at (cx + f x / z, cy - f y / z): world +y is up,
    image rows grow downwards."""
    cam = RasterCamera.look_at((0, 0, 3), width=96, height=96, color_mode=RasterColor.Rgb)
    img = _raster_one(cam, (0.3, 0.2, 0.0), (0.03, 0.03, 0.03))
    a = img[..., 3].astype(np.float64)
    ys, xs = np.mgrid[0:96, 0:96] + 0.5
    cxm, cym = (a * xs).sum() / a.sum(), (a * ys).sum() / a.sum()
    assert abs(cxm - (cam.cx + cam.fx * 0.3 / 3)) < 0.05
    assert abs(cym - (cam.cy - cam.fy * 0.2 / 3)) < 0.05


def _quat(axis, angle):
    axis = np.asarray(axis, np.float64) / np.linalg.norm(axis)
    return (math.cos(angle / 2), *(math.sin(angle / 2) * axis))


def test_raster_isotropic_rotation_invariance():
    cam = RasterCamera.look_at((0.4, 0.7, 2.5), width=80, height=64, color_mode=RasterColor.Rgb)
    ref = _raster_one(cam, (0.1, -0.05, 0.2), (0.08, 0.08, 0.08))
    rng = np.random.default_rng(3)
    for _ in range(4):
        q = rng.normal(size=4)
        got = _raster_one(cam, (0.1, -0.05, 0.2), (0.08, 0.08, 0.08), quat=tuple(q))
        np.testing.assert_allclose(got, ref, atol=2e-6)
    assert ref[..., 3].max() > 0.5


@pytest.mark.parametrize("theta", [0.0, 0.4, math.pi / 2, 2.2])
def test_raster_rotated_ellipse_conic(theta):
    """A flat ellipse (sx, sy, sz) on the optical axis turned by theta about the view axis: its 2D
    covariance is (f/z)^2 Rot(-theta) diag(sx^2, sy^2) Rot(-theta)^T + 0.3 I (image y points down, so
    the on-screen turn is -theta)."""
    cam = RasterCamera.look_at((0, 0, 3), width=96, height=80, color_mode=RasterColor.Rgb)
    sx, sy = 0.15, 0.04
    img = _raster_one(cam, (0, 0, 0), (sx, sy, 0.01), quat=_quat((0, 0, 1), theta), opacity=0.7)
    k = cam.fx / 3.0
    c, s = math.cos(-theta), math.sin(-theta)
    Rt = np.array([[c, -s], [s, c]])
    cov = k * k * Rt @ np.diag([sx * sx, sy * sy]) @ Rt.T
    alpha = _expected_alpha(cam, cov[0, 0] + 0.3, cov[0, 1], cov[1, 1] + 0.3, cam.cx, cam.cy, 0.7)
    np.testing.assert_allclose(img[..., 3], alpha, atol=3e-6)


def test_raster_axis_swap():
    """Scales (a, b, c) turned 90 degrees about the view axis draw the image of scales (b, a, c)."""
    cam = RasterCamera.look_at((0, 0, 3), width=64, height=64, color_mode=RasterColor.Rgb)
    turned = _raster_one(cam, (0, 0, 0), (0.12, 0.05, 0.02), quat=_quat((0, 0, 1), math.pi / 2))
    swapped = _raster_one(cam, (0, 0, 0), (0.05, 0.12, 0.02))
    np.testing.assert_allclose(turned, swapped, atol=2e-6)


def test_raster_front_to_back_compositing():
    """Two layers: rgb = c1 a1 + c2 a2 (1 - a1), alpha = 1 - (1 - a1)(1 - a2), the nearer first
    whatever the input order; at equal depth the lower index is in front."""
    cam = RasterCamera.look_at((0, 0, 3), width=48, height=48, color_mode=RasterColor.Rgb)
    near = ((0.0, 0.0, 0.5), (0.1, 0.1, 0.1), 0.6, (1.0, 0.0, 0.0))
    far = ((0.05, 0.0, -0.5), (0.12, 0.12, 0.12), 0.5, (0.0, 1.0, 0.0))

    def run(gs):
        pv = np.array([[*g[0], 1.0] for g in gs], f32)
        so = np.array([[*g[1], g[2]] for g in gs], f32)
        sh = np.array([g[3] for g in gs], f32)
        rot = np.tile(np.array([1, 0, 0, 0], f32), (len(gs), 1))
        return O.raster_gaussians_3d(pv, sh, rot, so, cam).astype(np.float64)

    a, b = run([near]), run([far])
    both = run([far, near])
    np.testing.assert_allclose(both, run([near, far]), atol=0)
    a1, a2 = a[..., 3], b[..., 3]
    np.testing.assert_allclose(both[..., 0], a[..., 0] + b[..., 0] * (1 - a1), atol=2e-6)
    np.testing.assert_allclose(both[..., 1], a[..., 1] + b[..., 1] * (1 - a1), atol=2e-6)
    np.testing.assert_allclose(both[..., 3], 1 - (1 - a1) * (1 - a2), atol=2e-6)
    tie = [((0, 0, 0), (0.1, 0.1, 0.1), 0.6, (1.0, 0.0, 0.0)), ((0, 0, 0), (0.1, 0.1, 0.1), 0.6, (0.0, 0.0, 1.0))]
    t = run(tie)
    assert t[24, 24, 0] > t[24, 24, 2] > 0  # index 0 (red) in front


def test_raster_transmittance_cut():
    """Layers of alpha 0.95: T runs 0.05, 0.0025, 1.25e-4; the fourth would take it below 1e-4,
    so the pixel stops after three."""
    cam = RasterCamera.look_at((0, 0, 3), width=32, height=32, color_mode=RasterColor.Rgb)
    n = 6
    pv = np.array([[0, 0, 0.1 * k, 1.0] for k in range(n)], f32)
    so = np.array([[0.5, 0.5, 0.5, 0.95]] * n, f32)  # wide: alpha ~ 0.95 across the centre pixels
    sh = np.array([[1.0, 1.0, 1.0]] * n, f32)
    rot = np.tile(np.array([1, 0, 0, 0], f32), (n, 1))
    img = O.raster_gaussians_3d(pv, sh, rot, so, cam)
    # each layer alone, nearest first (layer k sits at depth 3 - 0.1 k)
    a = [np.float64(O.raster_gaussians_3d(pv[k:k + 1], sh[:1], rot[:1], so[:1], cam)[16, 16, 3])
         for k in range(n - 1, -1, -1)]
    assert all(0.9 < x <= 0.95 for x in a)
    t3 = (1 - a[0]) * (1 - a[1]) * (1 - a[2])
    assert t3 >= 1e-4 > t3 * (1 - a[3])  # three layers pass the cut, the fourth would not
    assert abs(img[16, 16, 3] - (1 - t3)) < 1e-6
    assert abs(img[16, 16, 0] - (1 - t3)) < 1e-6


def _sh_basis_scipy(lmax, d):
    """Real spherical harmonics with the Condon-Shortley phase, index l^2 + l + m:
    m < 0: sqrt2 Im Y_l^|m|, m = 0: Y_l^0, m > 0: sqrt2 Re Y_l^m (scipy's complex Y_l^m)."""
    from scipy.special import sph_harm_y

    x, y, z = d
    polar, azim = math.acos(max(-1.0, min(1.0, z))), math.atan2(y, x)
    out = []
    for l in range(lmax + 1):
        for m in range(-l, l + 1):
            Y = complex(sph_harm_y(l, abs(m), polar, azim))
            out.append(math.sqrt(2) * Y.imag if m < 0 else (Y.real if m == 0 else math.sqrt(2) * Y.real))
    return np.array(out)


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_raster_sh_basis_against_scipy(degree):
    """Colour = max(0, sum_k basis_k(view direction) coef_k + 0.5), read back as rgb / alpha at the
    Gaussian's centre pixel, for each basis function alone."""
    K = (degree + 1) ** 2
    eye = (0.6, -0.4, 2.2)
    cam = RasterCamera.look_at(eye, width=32, height=32, sh_degree=degree)
    rng = np.random.default_rng(degree)
    p = rng.uniform(-0.05, 0.05, 3)
    centre = np.array(eye)
    d = (p.astype(f32).astype(np.float64) - centre)
    d /= np.linalg.norm(d)
    basis = _sh_basis_scipy(degree, d)
    for k in range(K):
        coef = np.zeros((K, 3), f32)
        coef[k] = (0.8, -0.8, 0.3)
        img = _raster_one(cam, tuple(p), (0.3, 0.3, 0.3), opacity=0.5, sh=coef.ravel())
        px = img[16, 16].astype(np.float64)
        want = np.maximum(basis[k] * np.array([0.8, -0.8, 0.3]) + 0.5, 0.0)
        np.testing.assert_allclose(px[:3] / px[3], want, atol=2e-5, err_msg=f"coefficient {k}")


def test_raster_culling():
    """Hidden (visibility 0), behind the camera, beyond the far plane: nothing is drawn."""
    cam = RasterCamera.look_at((0, 0, 3), width=32, height=32, far_plane=10.0, color_mode=RasterColor.Rgb)
    for pos, vis in (((0, 0, 0), 0.0), ((0, 0, 4), 1.0), ((0, 0, -8), 1.0)):
        pv = np.array([[*pos, vis]], f32)
        img = O.raster_gaussians_3d(pv, np.ones(3, f32), np.array([[1, 0, 0, 0]], f32),
                                    np.array([[0.2, 0.2, 0.2, 0.9]], f32), cam)
        assert not img.any()
    assert O.raster_gaussians_3d(np.zeros((0, 4), f32), np.zeros(0, f32), np.zeros((0, 4), f32),
                                 np.zeros((0, 4), f32), cam).sum() == 0
