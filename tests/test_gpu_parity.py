"""HIP path vs the CPU oracle on identical seeded inputs (runs on an MI355X).

Gates: hashgrid cell ids, sort order and neighbour
lists bit-exact; single step within 1e-5 (norm-relative); 64-step rollout within
1e-3; decoded images within 0.5 dB PSNR of the CPU image.
"""
import numpy as np
import pytest

from burn_automata_amd import kernels as K
from burn_automata_amd.config import (Boundary, GaussianDecodeConfig, GaussianDecodeMode,
                                      HashGridConfig, HashGridMode, NpaConfig, PerceptionOptions,
                                      Splat2dConfig)
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from burn_automata_amd import synthetic as syn
from oracle import oracle as O
from tests.helpers import psnr, rel_err, to_np

pytestmark = pytest.mark.gpu

STEP_TOL = 1e-5
ROLLOUT_TOL = 1e-3


def _hashgrid_cases():
    c1_model, c1_grid = syn.config_c1()
    cases = {
        "c1_4096": (syn.uniform_disk(4096, 42), 1, 4096, c1_grid),
        "c2_65536": (syn.uniform_disk(65536, 42), 1, 65536, c1_grid),
        "growing_2d_tiny": (np.array([[-0.9, -0.9, 0, 0], [0.9, 0.9, 0, 0]], np.float32), 1, 2,
                            HashGridConfig.growing_2d().replace(grid_size=(4, 4, 1))),
        "texture_2d_periodic": (syn.uniform_disk(1000, 7, radius=1.5), 1, 1000,
                                HashGridConfig.texture_2d()),
        "grid_clamped": (syn.uniform_disk(777, 9, radius=2.0), 1, 777,
                         HashGridConfig(2, Boundary.Clamped, HashGridMode.Grid, (12, 9, 1), 0.15)),
        "growing_3dgs": (syn.uniform_ball(3000, 5, radius=0.6), 1, 3000,
                         HashGridConfig.growing_3dgs()),
        "batch3": (np.concatenate([syn.uniform_disk(500, 11 + k) for k in range(3)]), 3, 500,
                   c1_grid),
        "skewed_gmm": (syn.gaussian_mixture(20000, 3), 1, 20000, c1_grid),
        "single_cell": (np.zeros((300, 4), np.float32), 1, 300, c1_grid),
        # a bin count that is not a multiple of four, in several systems
        "batch_odd_cells": (np.concatenate([syn.uniform_disk(400, 61 + k, radius=1.2) for k in range(3)]), 3, 400,
                            HashGridConfig(2, Boundary.Clamped, HashGridMode.Grid, (7, 5, 1), 0.3)),
        # Particle-mode bins shared by several true cells: 2-8 cells per bin (the split reorders
        # them), more than 8 (the bin keeps the reference order), and sparse bins (one lane per bin)
        "collide_reorder": (syn.uniform_disk(4000, 51, radius=0.5), 1, 4000,
                            c1_grid.replace(grid_size=(8, 8, 1))),
        "collide_keep": (syn.uniform_disk(4000, 52, radius=0.6), 1, 4000,
                         c1_grid.replace(grid_size=(4, 4, 1))),
        "collide_sparse": (syn.uniform_disk(300, 53, radius=1.0), 1, 300,
                           c1_grid.replace(grid_size=(16, 16, 1))),
        "collide_3d": (syn.uniform_ball(3000, 54, radius=0.6), 1, 3000,
                       HashGridConfig.growing_3dgs().replace(grid_size=(8, 8, 8))),
    }
    return cases


@pytest.mark.parametrize("name", list(_hashgrid_cases().keys()))
def test_hashgrid_bit_exact(ctx, name):
    pos, b, n, cfg = _hashgrid_cases()[name]
    want = O.build_hashgrid(pos, b, n, cfg)
    got = K.build_hashgrid(pos, b, n, cfg, ctx=ctx)
    np.testing.assert_array_equal(to_np(got.bin_offsets).astype(np.uint32), want.bin_offsets)
    np.testing.assert_array_equal(to_np(got.permutation).astype(np.uint32), want.permutation)
    np.testing.assert_array_equal(to_np(got.inverse_permutation).astype(np.uint32),
                                  want.inverse_permutation)


@pytest.mark.parametrize("name", ["c1_4096", "texture_2d_periodic", "grid_clamped",
                                  "growing_3dgs", "batch3", "skewed_gmm", "single_cell",
                                  "collide_reorder", "collide_keep", "collide_sparse", "collide_3d"])
def test_neighbor_lists_bit_exact(ctx, name):
    pos, b, n, cfg = _hashgrid_cases()[name]
    off_w, idx_w = O.neighbor_lists(pos, b, n, cfg)
    off_g, idx_g = K.neighbor_lists(pos, b, n, cfg, ctx=ctx)
    np.testing.assert_array_equal(to_np(off_g).astype(np.uint32), off_w)
    np.testing.assert_array_equal(to_np(idx_g).astype(np.uint32), idx_w)


def test_known_answer_sph_constants(ctx):
    """perceive_matches_upstream_sph_kernel_constants (crates/burn_automata_kernels/src/lib.rs:100-120)."""
    cfg = HashGridConfig.growing_2d().replace(grid_size=(4, 4, 1), eps=0.1)
    pos = np.array([[0, 0, 0, 0], [0.05, 0, 0, 0]], np.float32)
    st = np.array([1, 0, 0, 1], np.float32)
    out = K.perceive(pos, st, 1, 2, 2, cfg, True, True, ctx=ctx)
    d = to_np(out.density)
    blur = to_np(out.blurred_state).ravel()
    sg = to_np(out.state_gradient).ravel()
    dg = to_np(out.density_gradient).ravel()
    assert abs(d[0] - 181.03874) <= 1e-3 and abs(d[1] - 181.03874) <= 1e-3
    for k, v in enumerate([0.7032967, 0.2967033, 0.2967033, 0.7032967]):
        assert abs(blur[k] - v) <= 1e-5
    assert abs(sg[0] + 13.186813) <= 1e-4 and abs(sg[2] - 13.186813) <= 1e-4
    assert abs(dg[0] - 1193.662) <= 1e-3 and abs(dg[2] + 1193.662) <= 1e-3


def _perceive_cases():
    c1_model, c1_grid = syn.config_c1()
    n = 4096
    pos = syn.uniform_disk(n, 42)
    st = syn.normal_states(n, 16, 42)
    base = c1_model.perception_options()
    return {
        "c1_branch_b": (pos, st, 1, n, 16, c1_grid, base),
        "c1_branch_a": (pos, st, 1, n, 16, c1_grid,
                        c1_model.replace(density_grad=True).perception_options()),
        "no_lognorm_eps_scaled": (pos, st, 1, n, 16, c1_grid.replace(eps=0.07),
                                  PerceptionOptions(True, True, 0.05, True, True, False, False,
                                                    True, True)),
        "state_only": (pos, st, 1, n, 16, c1_grid, PerceptionOptions(False, False, 0.05)),
        "dgrad_only": (pos, st, 1, n, 16, c1_grid,
                       PerceptionOptions(False, True, 0.05, log_norm_density_grad=True)),
        "texture_periodic_s5": (syn.uniform_disk(1500, 3, radius=1.0),
                                syn.normal_states(1500, 5, 3), 1, 1500, 5,
                                HashGridConfig.texture_2d(),
                                NpaConfig.texture_2d().perception_options()),
        "growing_3d": (syn.uniform_ball(2500, 8, radius=0.5), syn.normal_states(2500, 24, 8), 1,
                       2500, 24, HashGridConfig.growing_3dgs(),
                       NpaConfig.growing_3dgs().perception_options()),
        "batch2_s8": (np.concatenate([syn.uniform_disk(800, 1), syn.uniform_disk(800, 2)]),
                      syn.normal_states(1600, 8, 4), 2, 800, 8, c1_grid,
                      NpaConfig.growing_2d().replace(state_dims=8, eps0=0.05).perception_options()),
    }


def _dense_cell_case(dim, n_dense, n_rest, seed):
    """A cell far denser than its neighbours: targets around it visit more neighbour chunks
    (runs of <= 64 slots) than the density pass records, so their items take the second pass's
    own candidate tests, while the other items build their lists from the recorded masks."""
    rng = np.random.default_rng(seed)
    if dim == 2:
        cfg = syn.config_c1()[1]
        rest = syn.uniform_disk(n_rest, seed, radius=0.4)
    else:
        cfg = HashGridConfig.growing_3dgs()
        rest = syn.uniform_ball(n_rest, seed, radius=0.5)
    lo, hi = 0.2 * cfg.eps, 0.8 * cfg.eps  # strictly inside the cell [0, eps)^dim
    dense = np.zeros((n_dense, 4), np.float32)
    dense[:, :dim] = rng.uniform(lo, hi, size=(n_dense, dim)).astype(np.float32)
    pos = np.concatenate([dense, rest]).astype(np.float32)
    pos = pos[rng.permutation(len(pos))]  # dense particles spread over the index range
    return pos, cfg


@pytest.mark.parametrize("dim,n_dense,n_rest", [(2, 1800, 3000), (3, 3400, 3000)])
def test_perceive_dense_cell_bit_exact(ctx, dim, n_dense, n_rest):
    pos, cfg = _dense_cell_case(dim, n_dense, n_rest, 5 + dim)
    n = len(pos)
    S = 16 if dim == 2 else 24
    st = syn.normal_states(n, S, 9)
    opts = (syn.config_c1()[0] if dim == 2 else NpaConfig.growing_3dgs()).perception_options()
    want = O.perceive_with_options(pos, st, 1, n, S, cfg, opts)
    got = K.perceive_with_options(pos, st, 1, n, S, cfg, opts, ctx=ctx)
    np.testing.assert_array_equal(to_np(got.density), want.density)
    np.testing.assert_array_equal(to_np(got.features), want.features)


@pytest.mark.parametrize("name", list(_perceive_cases().keys()))
def test_perceive_parity(ctx, name):
    pos, st, b, n, S, cfg, opts = _perceive_cases()[name]
    want = O.perceive_with_options(pos, st, b, n, S, cfg, opts)
    got = K.perceive_with_options(pos, st, b, n, S, cfg, opts, ctx=ctx)
    assert got.feature_dims == want.feature_dims
    np.testing.assert_array_equal(to_np(got.density), want.density)
    for field in ("features", "blurred_state", "state_gradient", "density_gradient"):
        e = rel_err(getattr(got, field), getattr(want, field))
        assert e <= STEP_TOL, f"{field}: {e}"


def _model_case(name):
    if name == "c1":
        w = syn.workload("c1")
        return w["model"], w["grid"], w["positions"], w["states"], w["weights"], 1, w["n"]
    if name == "c1_dgrad":
        w = syn.workload("c1_dgrad")
        return w["model"], w["grid"], w["positions"], w["states"], w["weights"], 1, w["n"]
    if name == "growing_3d":
        m = NpaConfig.growing_3dgs()
        g = HashGridConfig.growing_3dgs()
        n = 2048
        return (m, g, syn.uniform_ball(n, 4, 0.5), syn.normal_states(n, m.state_dims, 4),
                syn.seeded_weights(m, 4), 1, n)
    if name == "torus_gates_3d":
        m = NpaConfig.torus_field_3dgs()
        g = HashGridConfig.growing_3dgs()
        n = 1024
        pos = syn.uniform_ball(n, 6, 0.5)
        pos[::7, 3] = 1.0  # anchored particles
        st = syn.normal_states(n, m.state_dims, 6, std=1.0)
        st[:, 3] += 3.5
        return m, g, pos, st, syn.seeded_weights(m, 6), 1, n
    if name == "texture_periodic":
        m = NpaConfig.texture_2d()
        g = HashGridConfig.texture_2d()
        n = 1500
        return (m, g, syn.uniform_disk(n, 12, 1.0), syn.normal_states(n, 16, 12),
                syn.seeded_weights(m, 12), 1, n)
    if name == "batch4":
        m, g = syn.config_c1()
        n = 1024
        pos = np.concatenate([syn.uniform_disk(n, 20 + k) for k in range(4)])
        return m, g, pos, syn.normal_states(4 * n, 16, 20), syn.seeded_weights(m, 20), 4, n
    if name == "texture_periodic_common":  # the rollout's usual options on a periodic grid: the
        # fused kernel's periodic variant (wrapped deltas and positions compiled in)
        m = NpaConfig.texture_2d().replace(density_grad=False)
        g = HashGridConfig.texture_2d()
        n = 1500
        return (m, g, syn.uniform_disk(n, 14, 1.0), syn.normal_states(n, 16, 14),
                syn.seeded_weights(m, 14), 1, n)
    if name == "no_sgrad_2d":  # density gradient and positions without the state gradient, H < 128
        m = NpaConfig(eps0=0.05, hidden_dims=96, state_grad=False, density_grad=True,
                      position_features=True)
        _, g = syn.config_c1()
        n = 3000
        return (m, g, syn.uniform_disk(n, 31, 0.6), syn.normal_states(n, 16, 31),
                syn.seeded_weights(m, 31), 1, n)
    if name == "no_sgrad_3d":  # 24 channels: the two-kernel path
        m = NpaConfig.torus_field_3dgs().replace(state_grad=False)
        g = HashGridConfig.growing_3dgs()
        n = 1024
        return (m, g, syn.uniform_ball(n, 32, 0.5), syn.normal_states(n, m.state_dims, 32),
                syn.seeded_weights(m, 32), 1, n)
    if name == "torus16_gates_3d":  # 16 channels, density gradient, positions, 3D gates
        m = NpaConfig.torus_field_3dgs().replace(state_dims=16, hidden_dims=128)
        g = HashGridConfig.growing_3dgs()
        n = 1024
        pos = syn.uniform_ball(n, 33, 0.5)
        pos[::5, 3] = 1.0  # anchored particles
        st = syn.normal_states(n, m.state_dims, 33, std=1.0)
        st[:, 3] += 3.5
        return m, g, pos, st, syn.seeded_weights(m, 33), 1, n
    if name in ("collide_reorder", "collide_keep", "collide_sparse", "collide_3d"):
        pos, b, n, g = _hashgrid_cases()[name]
        m = NpaConfig.growing_3dgs() if g.dim == 3 else syn.config_c1()[0]
        return (m, g, pos, syn.normal_states(n, m.state_dims, 60), syn.seeded_weights(m, 60), b, n)
    raise KeyError(name)


@pytest.mark.parametrize("name", ["c1", "c1_dgrad", "growing_3d", "torus_gates_3d",
                                  "texture_periodic", "texture_periodic_common", "batch4",
                                  "no_sgrad_2d", "no_sgrad_3d",
                                  "torus16_gates_3d", "collide_reorder", "collide_keep",
                                  "collide_sparse", "collide_3d"])
def test_step_parity(ctx, name):
    """One step against NpaModel::step_cpu (model.rs:768-858). 16-channel models run the fused
    second-pass + MLP kernel, wider ones the two-kernel path; both sum in the reference's order."""
    m, g, pos, st, w, b, n = _model_case(name)
    mask = O.update_mask(b, n, 0.5, 0, 42)
    want = O.step(m, w, pos, st, b, n, g, 1.0, mask)
    got = NpaModel(m, w).step(pos, st, b, n, g, 1.0, update_mask=mask, ctx=ctx)
    assert rel_err(got.density, want.density) <= STEP_TOL
    assert rel_err(got.next_positions, want.next_positions) <= STEP_TOL
    assert rel_err(got.next_states, want.next_states) <= STEP_TOL
    np.testing.assert_array_equal(to_np(got.density), want.density)
    np.testing.assert_array_equal(to_np(got.next_positions), want.next_positions)
    np.testing.assert_array_equal(to_np(got.next_states), want.next_states)


def test_mlp_forward_parity(ctx):
    m, g, pos, st, w, b, n = _model_case("c1")
    feats = O.perceive_with_options(pos, st, b, n, m.state_dims, g, m.perception_options()).features
    want_dx, want_ds = O.forward_from_features_with_eps(m, w, feats, g.eps)
    dx, ds = NpaModel(m, w).forward_from_features_with_eps(feats, g.eps, ctx=ctx)
    assert rel_err(dx, want_dx) <= STEP_TOL
    assert rel_err(ds, want_ds) <= STEP_TOL


def test_euler_step_parity(ctx):
    n, S = 3000, 9
    rng = np.random.default_rng(0)
    pos = rng.normal(size=(n, 4)).astype(np.float32)
    st = rng.normal(size=(n, S)).astype(np.float32) * 10
    dx = rng.normal(size=(n, 4)).astype(np.float32)
    ds = rng.normal(size=(n, S)).astype(np.float32) * 10
    mask = (rng.random(n) < 0.5).astype(np.float32)
    for cfg in (HashGridConfig.growing_2d(), HashGridConfig.texture_2d(),
                HashGridConfig.growing_3dgs()):
        wp, ws = O.euler_step(pos, st, dx, ds, 1, n, S, cfg, 0.7, mask)
        gp, gs = K.euler_step(pos, st, dx, ds, 1, n, S, cfg, 0.7, mask, ctx=ctx)
        np.testing.assert_array_equal(to_np(gp), wp)
        np.testing.assert_array_equal(to_np(gs), ws)


def test_update_mask_bit_exact(ctx):
    for (b, n, p, step, seed) in [(1, 4096, 0.5, 0, 42), (3, 777, 0.3, 17, 2 ** 40 + 5),
                                  (2, 100, 1.0, 3, 1), (2, 100, 0.0, 3, 1)]:
        want = O.update_mask(b, n, p, step, seed)
        got = K.update_mask(b, n, p, step, seed, ctx=ctx)
        np.testing.assert_array_equal(to_np(got), want)


@pytest.mark.parametrize("name", ["c1", "batch4"])
def test_executor_rollout_64_steps(ctx, name):
    m, g, pos, st, w, b, n = _model_case(name)
    steps = 64
    want_p, want_s = O.rollout(m, w, pos, st, b, n, g, steps, 1.0, 0.5, 42, 0)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, 0.5, 42)
    ex.step_state_many(state, steps)
    gp, gs, _ = ex.read_state(state)
    assert state.step_index() == steps
    ep, es = rel_err(gp, want_p), rel_err(gs, want_s)
    print(f"{name}: 64-step rollout rel err pos={ep:.3e} state={es:.3e}")
    assert ep <= ROLLOUT_TOL and es <= ROLLOUT_TOL
    # the VALU engine sums in the reference's order: the rollout is the oracle's bit for bit
    np.testing.assert_array_equal(to_np(gp), want_p)
    np.testing.assert_array_equal(to_np(gs), want_s)


def test_rollout_trace_with_mean_dx(ctx):
    """run_rollout_from_particles (rollout/mod.rs:222-297): the final particles are the oracle
    rollout's bit for bit and each step's mean_dx is the serial f32 mean of the oracle step's
    motion norms over every particle, masked or not (rollout/mod.rs:277-283), within the
    single-step tolerance (the trace's MLP pass goes through npa_mlp_forward)."""
    from burn_automata_amd.config import RolloutConfig
    from burn_automata_amd.rollout import mean_dx_norm, run_rollout_from_particles
    m, g, pos, st, w, b, n = _model_case("batch4")
    cfg = RolloutConfig(batch_size=b, particle_count=n, steps=6, dt=1.0, update_prob=0.5, seed=42)
    trace = run_rollout_from_particles(NpaModel(m, w), g, cfg, pos, st,
                                       executor=HipAutomataExecutor(ctx=ctx))
    p, s, want = pos, st, []
    for k in range(cfg.steps):
        out = O.step(m, w, p, s, b, n, g, cfg.dt, O.update_mask(b, n, cfg.update_prob, k, cfg.seed))
        want.append(mean_dx_norm(out.dx))
        p, s = out.next_positions, out.next_states
    np.testing.assert_array_equal(to_np(trace.positions), p)
    np.testing.assert_array_equal(to_np(trace.states), s)
    assert len(trace.mean_dx) == cfg.steps and min(want) > 0
    np.testing.assert_allclose(trace.mean_dx, want, rtol=STEP_TOL, atol=0)
    fast = run_rollout_from_particles(NpaModel(m, w), g, cfg, pos, st,
                                      executor=HipAutomataExecutor(ctx=ctx), record_mean_dx=False)
    assert fast.mean_dx == []
    np.testing.assert_array_equal(to_np(fast.positions), p)


def test_state_outlives_its_context():
    """A state keeps its context alive: the state still steps and reads after the caller destroyed
    the context, and destroying the state last releases both (no use of freed memory)."""
    from burn_automata_amd._lib import lib
    from burn_automata_amd.runtime import Context
    m, g, pos, st, w, b, n = _model_case("c1")
    c = Context(0)
    ex = HipAutomataExecutor(ctx=c)
    state = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, 0.5, 42)
    ex.step_state(state)
    want_p, want_s, _ = ex.read_state(state)
    c.close()
    assert lib().npa_state_step(state.handle, 1) == 0
    state.close()
    assert want_p.shape[0] == b * n and np.isfinite(to_np(want_s)).all()


def test_executor_single_steps_match_fused_step(ctx):
    m, g, pos, st, w, b, n = _model_case("c1")
    ex = HipAutomataExecutor(ctx=ctx)
    model = NpaModel(m, w)
    state = ex.create_state(model, pos, st, b, n, g, 1.0, 0.5, 42)
    p, s = pos, st
    for k in range(3):
        mask = K.update_mask(b, n, 0.5, k, 42, ctx=ctx)
        out = model.step(p, s, b, n, g, 1.0, update_mask=mask, ctx=ctx)
        p, s = out.next_positions, out.next_states
        ex.step_state(state)
    gp, gs, gd = ex.read_state(state)
    np.testing.assert_array_equal(to_np(gp), to_np(p))
    np.testing.assert_array_equal(to_np(gs), to_np(s))
    np.testing.assert_array_equal(to_np(gd), to_np(out.density))


def test_update_probability_zero_keeps_state(ctx):
    """wgpu_update_probability_zero_keeps_state_fixed (tests/gpu_wgpu/updates.rs:4-33)."""
    m, g, pos, st, w, b, n = _model_case("c1")
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, 0.0, 53)
    ex.step_state(state)
    gp, gs, _ = ex.read_state(state)
    np.testing.assert_array_equal(to_np(gp), pos)
    np.testing.assert_array_equal(to_np(gs), st)


@pytest.mark.parametrize("name", ["texture_periodic", "texture_periodic_common", "torus_gates_3d"])
def test_masked_particles_follow_the_cpu_euler_step(ctx, name):
    """Particles with update mask 0 skip the second pass and the MLP on the device; the CPU
    euler_step (step.rs:4-55) still wraps their positions on a periodic grid and clamps their 3D
    opacity logits. Both step paths must equal the oracle bit for bit, masked particles included."""
    m, g, pos, st, w, b, n = _model_case(name)
    if g.dim == 3:  # opacity logits outside [-8, 24] on masked and unmasked particles
        st = st.copy()
        st[::3, 3] = 30.0
        st[1::5, 8] = -20.0
    if name.startswith("texture_periodic"):  # particles beyond the periodic extent and at its edges
        pos = pos.copy()
        half = 0.5 * g.grid_size[0] * g.eps
        pos[::11, 0] = np.float32(half * 1.37)
        pos[::13, 1] = np.float32(-half)
    mask = O.update_mask(b, n, 0.5, 3, 42)
    assert 0 < mask.sum() < mask.size
    want = O.step(m, w, pos, st, b, n, g, 1.0, mask)
    got = NpaModel(m, w).step(pos, st, b, n, g, 1.0, update_mask=mask, ctx=ctx)
    np.testing.assert_array_equal(to_np(got.next_positions), want.next_positions)
    np.testing.assert_array_equal(to_np(got.next_states), want.next_states)
    held = mask == 0  # the case exercises the transform: some held values are not their inputs
    assert ((want.next_positions[held] != pos[held]).any()
            or (want.next_states[held] != st[held]).any())
    want_p, want_s = O.rollout(m, w, pos, st, b, n, g, 4, 1.0, 0.5, 42, 0)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, 0.5, 42)
    ex.step_state_many(state, 4)
    gp, gs, _ = ex.read_state(state)
    np.testing.assert_array_equal(to_np(gp), want_p)
    np.testing.assert_array_equal(to_np(gs), want_s)
    state.close()


@pytest.mark.parametrize("name,prob", [("c1", 0.5), ("growing_3d", 0.3), ("batch4", 1.0)])
def test_work_counters_match_oracle(ctx, name, prob):
    """npa_state_pair_counts (the bench's work counts): candidates and pairs of the density pass
    over every particle and of the update mask's targets, against the oracle's hashgrid bins,
    neighbour lists and mask on the state's particles after one step."""
    from tests.test_oracle import cell_coords_ref, cell_index_ref

    m, g, pos, st, w, b, n = _model_case(name)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, prob, 42)
    ex.step_state(state)  # the counters describe step 1, a nonzero step index
    got = ex.work_counts(state)
    p1 = to_np(ex.read_state(state)[0])
    cells = g.cell_count()
    sizes = np.diff(O.build_hashgrid(p1, b, n, g).bin_offsets.astype(np.int64))
    off, _ = O.neighbor_lists(p1, b, n, g)
    pairs = np.diff(off.astype(np.int64))
    zs = (-1, 0, 1) if g.dim == 3 else (0,)
    cand = np.zeros(b * n, np.int64)
    for i in range(b * n):
        c = cell_coords_ref(p1[i], g)
        for dz in zs:
            for dy in (-1, 0, 1):
                for dx in (-1, 0, 1):
                    cell = cell_index_ref((c[0] + dx, c[1] + dy, c[2] + dz), g)
                    if cell is not None:
                        cand[i] += sizes[(i // n) * cells + cell]
    mask = O.update_mask(b, n, prob, 1, 42) != 0
    want = {"candidates": int(cand.sum()), "pairs": int(pairs.sum()), "targets": int(mask.sum()),
            "target_candidates": int(cand[mask].sum()), "target_pairs": int(pairs[mask].sum())}
    assert got == want
    state.close()


def test_update_model_changes_trajectory(ctx):
    m, g, pos, st, w, b, n = _model_case("c1")
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, 1.0, 1)
    w2 = {k: v * 0.5 for k, v in w.items()}
    ex.update_state_model(state, w2)
    ex.step_state(state)
    gp, gs, _ = ex.read_state(state)
    want = O.step(m, w2, pos, st, b, n, g, 1.0, None)
    assert rel_err(gp, want.next_positions) <= STEP_TOL
    assert rel_err(gs, want.next_states) <= STEP_TOL


@pytest.mark.parametrize("mode", list(GaussianDecodeMode))
def test_decode_gaussians_parity(ctx, mode):
    n, S = 2000, 20
    rng = np.random.default_rng(1)
    pos = rng.normal(size=(n, 4)).astype(np.float32)
    st = rng.normal(size=(n, S)).astype(np.float32)
    cfg = GaussianDecodeConfig(mode=mode, sh_degree=1 if mode == GaussianDecodeMode.GaussianSh0Oriented else 0)
    want = O.decode_gaussians_3d(pos, st, S, cfg)
    got = K.decode_gaussians_3d(pos, st, S, cfg, ctx=ctx)
    for k in want:
        assert rel_err(got[k], want[k]) <= 1e-6, k


@pytest.mark.parametrize("size,sigma,n", [(64, 1.0, 512), (512, 0.004 * 511 / 2, 65536),
                                         (100, 3.0, 3000)])
def test_splat_psnr(ctx, size, sigma, n):
    pos = syn.uniform_disk(n, 5, radius=1.1)
    st = syn.normal_states(n, 16, 5, std=0.3)
    colors = O.tail_colors(st, 16)
    cfg = Splat2dConfig(image_size=size, sigma=sigma, pixel_size=2.0 / size)
    want = O.splat_particles_2d(pos, colors, cfg)
    got = K.splat_particles_2d(pos, colors, cfg, ctx=ctx)
    p = psnr(got, want)
    print(f"splat {size} psnr={p:.1f} dB rel={rel_err(got, want):.2e}")
    assert p >= 100.0
    assert rel_err(got, want) <= 1e-5


def test_state_splat_matches_oracle_image(ctx):
    m, g, pos, st, w, b, n = _model_case("c1")
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, 0.5, 42)
    cfg = Splat2dConfig(image_size=128, sigma=1.0, pixel_size=2.0 / 128)
    img = ex.splat_2d(state, cfg)
    want = O.splat_particles_2d(pos, O.tail_colors(st, 16), cfg)
    assert rel_err(img, want) <= 1e-5


def test_error_behaviour(ctx):
    from burn_automata_amd import _abi
    pos = syn.uniform_disk(10, 1)
    with pytest.raises(_abi.InvalidDim):
        K.build_hashgrid(pos, 1, 10, HashGridConfig.growing_2d().replace(dim=4), ctx=ctx)
    with pytest.raises(_abi.InvalidEps):
        K.build_hashgrid(pos, 1, 10, HashGridConfig.growing_2d().replace(eps=0.0), ctx=ctx)
    with pytest.raises(_abi.ParticleModeRequiresPowerOfTwo):
        K.build_hashgrid(pos, 1, 10, HashGridConfig.growing_2d().replace(grid_size=(6, 8, 1)),
                         ctx=ctx)
    with pytest.raises(_abi.InvalidGridSize):
        K.build_hashgrid(pos, 1, 10, HashGridConfig.growing_2d().replace(grid_size=(0, 8, 1)),
                         ctx=ctx)
    with pytest.raises(_abi.PositionShape):
        K.build_hashgrid(pos, 1, 11, HashGridConfig.growing_2d(), ctx=ctx)
    m, g = syn.config_c1()
    with pytest.raises(_abi.InvalidArgument):
        NpaModel(m, syn.seeded_weights(m)).step(pos, syn.normal_states(10, 16), 1, 10,
                                                HashGridConfig.growing_3dgs(), 1.0, ctx=ctx)
