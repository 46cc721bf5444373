"""The perception adjoint on the HIP path (npa_perceive_adjoint) against the CPU oracle.

npa_perceive_adjoint replaces perceive_adjoint_with_options
(crates/burn_automata_kernels/src/reference/adjoint.rs:27-136). The reference scatters each pair's
terms into both particles in its serial order; the device gathers them per particle over its own
neighbour list, so the sums are added in another order. Bar: max |GPU - CPU| <= 1e-4 of the
output's largest magnitude (state and position adjoints separately); measured in the 1e-6 range.
The reference's own finite-difference tests (lib.rs:123-356) are run on the device result too.
"""
import numpy as np
import pytest

from burn_automata_amd import _abi
from burn_automata_amd import kernels as K
from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import Boundary, HashGridConfig, HashGridMode, PerceptionOptions
from oracle import oracle as O
from tests.helpers import rel_err, to_np

pytestmark = pytest.mark.gpu

TOL = 1e-4
f32 = np.float32


def _compare(got, want, what):
    es = rel_err(got.state, want.state)
    ep = rel_err(to_np(got.position), want.position)
    print(f"{what}: state rel err {es:.2e}, position rel err {ep:.2e}")
    assert es <= TOL and ep <= TOL, what


def _fixture(eps):
    cfg = HashGridConfig(3, Boundary.Clamped, HashGridMode.Particle, (8, 8, 8), eps, 16)
    st = np.array([0.10, -0.20, 0.05, 0.30, 0.15, -0.10, -0.25, 0.35, 0.20, 0.05, -0.30, 0.40], f32)
    return cfg, st


def _opts(cfg, hybrid, pf):
    return PerceptionOptions(state_grad=True, density_grad=True, eps0=cfg.eps, scale_equivariance=True,
                             particle_density_equivariance=True, log_norm_grad=True,
                             log_norm_density_grad=True, hybrid_state_gradient=hybrid, position_features=pf)


def _loss(pos, st, cfg, opts, fa):
    f = O.perceive_with_options(pos, st, 1, 4, 3, cfg, opts).features.astype(np.float64)
    return float((f.ravel() * fa.astype(np.float64)).sum())


@pytest.mark.parametrize("case", ["state", "position", "position_hybrid"])
def test_reference_finite_difference_fixtures(ctx, case):
    """lib.rs:123-198, 201-277, 280-356: the device adjoint meets the reference's bounds and agrees
    with the oracle's adjoint of the same fixture."""
    if case == "state":
        cfg, st = _fixture(0.35)
        pos = np.array([[0, 0, 0, 0], [0.12, 0.04, -0.03, 0], [-0.08, 0.10, 0.02, 0], [0.04, -0.09, 0.11, 0]], f32)
        opts = _opts(cfg, True, False)
        F = opts.feature_dims(3, 3)
        fa = (np.sin((np.arange(4 * F, dtype=f32) + f32(1)) * f32(0.017)) * f32(0.1)).astype(f32)
    else:
        cfg, st = _fixture(0.40)
        pos = np.array([[0, 0, 0, 0], [0.11, 0.03, -0.02, 0], [-0.07, 0.09, 0.04, 0], [0.05, -0.08, 0.10, 0]], f32)
        hybrid = case == "position_hybrid"
        opts = _opts(cfg, hybrid, True)
        F = opts.feature_dims(3, 3)
        k = np.arange(4 * F, dtype=f32) + f32(5.0 if hybrid else 3.0)
        fa = ((np.sin(k * f32(0.011)) * f32(0.03)) if hybrid else (np.cos(k * f32(0.013)) * f32(0.05))).astype(f32)
    got = K.perceive_adjoint_with_options(pos, st, 1, 4, 3, cfg, opts, fa, ctx=ctx)
    _compare(got, O.perceive_adjoint_with_options(pos, st, 1, 4, 3, cfg, opts, fa), f"fixture {case}")
    gs, gp = to_np(got.state), to_np(got.position)
    if case == "state":
        p, m = st.copy(), st.copy()
        p[4] += f32(1e-3)
        m[4] -= f32(1e-3)
        fd = (_loss(pos, p, cfg, opts, fa) - _loss(pos, m, cfg, opts, fa)) / 2e-3
        assert abs(gs[4] - fd) <= 2e-3
    else:
        particle, axis, tol = (2, 1, 2.5e-1) if case == "position_hybrid" else (1, 0, 7.5e-2)
        p, m = pos.copy(), pos.copy()
        p[particle, axis] += f32(1e-4)
        m[particle, axis] -= f32(1e-4)
        fd = (_loss(p, st, cfg, opts, fa) - _loss(m, st, cfg, opts, fa)) / 2e-4
        assert abs(gp[particle, axis] - fd) <= tol


CASES = {
    # name: (dim, boundary, mode, grid, eps, hybrid, state_grad, density_grad, log_norm, pos_features,
    #        particles, side of the region they fill)
    "2d_growing_particle": (2, Boundary.Clamped, HashGridMode.Particle, (64, 64, 1), 0.05, False, True, False, True, False, 3000, 1.1),
    "2d_hybrid_all": (2, Boundary.Clamped, HashGridMode.Particle, (64, 64, 1), 0.05, True, True, True, True, True, 3000, 1.1),
    "2d_periodic_grid": (2, Boundary.Periodic, HashGridMode.Grid, (40, 40, 1), 0.05, False, True, True, False, False, 8000, 2.0),
    "3d_hybrid_particle": (3, Boundary.Clamped, HashGridMode.Particle, (16, 16, 16), 0.12, True, True, True, True, True, 2500, 1.0),
    "3d_blur_only_grid": (3, Boundary.Clamped, HashGridMode.Grid, (16, 16, 16), 0.12, False, False, False, False, True, 2500, 1.0),
    "2d_tiny_periodic_grid": (2, Boundary.Periodic, HashGridMode.Grid, (2, 2, 1), 0.5, True, True, True, True, False, 150, 1.0),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("S", [3, 16])
def test_adjoint_matches_the_oracle(ctx, name, S):
    """About 20 neighbours per particle (the tiny periodic grid: every particle, several times over
    - its 3x3 cell offsets wrap onto the same cells)."""
    dim, bnd, mode, gs, eps, hyb, sg, dg, ln, pf, n, side = CASES[name]
    cfg = HashGridConfig(dim, bnd, mode, gs, eps, 32)
    rng = np.random.default_rng(len(name) * 7 + S)
    pos = np.zeros((n, 4), f32)
    if bnd == Boundary.Periodic:  # periodic cells cover [0, extent)
        pos[:, :dim] = rng.uniform(0.0, side, (n, dim)) * 0.999
    else:  # clamped cells are centred on the origin
        pos[:, :dim] = rng.uniform(-side / 2, side / 2, (n, dim))
    pos[:, 3] = rng.uniform(-1, 1, n)
    st = rng.normal(0, 0.5, n * S).astype(f32)
    opts = PerceptionOptions(state_grad=sg, density_grad=dg, eps0=eps * 0.8, scale_equivariance=True,
                             particle_density_equivariance=True, log_norm_grad=ln, log_norm_density_grad=ln,
                             hybrid_state_gradient=hyb, position_features=pf)
    F = opts.feature_dims(S, dim)
    fa = rng.normal(0, 0.1, n * F).astype(f32)
    want = O.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, fa)
    got = K.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, fa, ctx=ctx)
    _compare(got, want, f"{name} S={S}")
    again = K.perceive_adjoint_with_options(pos, st, 1, n, S, cfg, opts, fa, ctx=ctx)
    np.testing.assert_array_equal(to_np(again.state), to_np(got.state))  # deterministic
    np.testing.assert_array_equal(to_np(again.position), to_np(got.position))


def test_c1_model_adjoint_batched(ctx):
    """The growing-2D model's perception options on C1 particles, three systems in one batch."""
    w = syn.workload("c1", particles=2048)
    m, g = w["model"], w["grid"]
    opts = m.perception_options()
    B, n, S = 3, 2048, m.state_dims
    pos = np.concatenate([w["positions"]] * B)
    rng = np.random.default_rng(5)
    st = rng.normal(0, 0.3, B * n * S).astype(f32)
    F = opts.feature_dims(S, g.dim)
    fa = rng.normal(0, 0.1, B * n * F).astype(f32)
    want = O.perceive_adjoint_with_options(pos, st, B, n, S, g, opts, fa)
    got = K.perceive_adjoint_with_options(pos, st, B, n, S, g, opts, fa, ctx=ctx)
    _compare(got, want, "c1 batch 3")


def test_adjoint_errors(ctx):
    cfg, st = _fixture(0.35)
    pos = np.zeros((4, 4), f32)
    opts = _opts(cfg, True, False)
    with pytest.raises(_abi.OutputShape, match="does not match expected"):
        K.perceive_adjoint_with_options(pos, st, 1, 4, 3, cfg, opts, np.zeros(5, f32), ctx=ctx)
    with pytest.raises(_abi.InvalidEps):
        K.perceive_adjoint_with_options(pos, st, 1, 4, 3, cfg.replace(eps=-1.0), opts,
                                        np.zeros(4 * opts.feature_dims(3, 3), f32), ctx=ctx)
