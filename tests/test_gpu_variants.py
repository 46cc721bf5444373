"""Grid variants and the fused step kernel's compile-time variants against the CPU oracle (MI355X).

The fused second pass + MLP + Euler kernel is instantiated per spatial dimension D (2, 3), option
set FL (5: state gradient + hybrid moment, clamped; 13: the same on a periodic grid, wrapped deltas
and positions compiled in; -1: every option read at run time, e.g. with the density gradient) and
MLP engine (VALU bit-exact, matrix cores). Every instantiation runs here, on grids of every kind
(Grid or Particle mode, clamped or periodic, 2D and 3D) and on dense cells whose targets overflow
the density pass's recorded neighbour chunks and the fused kernel's LDS neighbour list.

Gates: the hashgrid, the neighbour lists, the Euler step and the VALU engine's step are bit-exact
against the oracle (hashgrid.rs:16-193, neighbor.rs:3-44, step.rs:4-55, model.rs:768-858); the
matrix-core engine's step is within the single-step gate 1e-5 with a bit-exact density.
"""
import numpy as np
import pytest

from burn_automata_amd import _abi
from burn_automata_amd import kernels as K
from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import Boundary, HashGridConfig, HashGridMode, NpaConfig
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from burn_automata_amd.runtime import Context
from oracle import oracle as O
from tests.helpers import rel_err, to_np

pytestmark = pytest.mark.gpu

STEP_TOL = 1e-5

P, C = Boundary.Periodic, Boundary.Clamped
GRID, PART = HashGridMode.Grid, HashGridMode.Particle

# name: (grid, particle count, cloud radius). Periodic clouds reach past the domain's half extent, so
# the wrapped cell index (Grid mode), the minimum-image delta and the position wrap all take part.
GRIDS = {
    "grid3_periodic": (HashGridConfig(3, P, GRID, (10, 9, 8), 0.1), 3000, 0.6),
    "particle3_periodic": (HashGridConfig(3, P, PART, (16, 16, 8), 0.1), 3000, 0.5),
    "grid3_clamped": (HashGridConfig(3, C, GRID, (10, 9, 8), 0.1), 3000, 0.6),
    "particle2_periodic": (HashGridConfig(2, P, PART, (16, 16, 1), 0.05), 3000, 0.45),
    "grid2_periodic_small": (HashGridConfig(2, P, GRID, (6, 5, 1), 0.1), 1500, 0.4),
    # strips longer than the grid along x (radius < 0: half length 2, half width 0.3): coordinate bins
    # hold two cells there, so the sort marks those bins unsplit and the passes filter by cell; sparse
    # grids (more cells than particles) take the small-system build and the four-lane density passes
    "particle2_strip_sparse": (HashGridConfig(2, C, PART, (64, 64, 1), 0.05), 3000, -1.0),
    "particle3_strip_sparse": (HashGridConfig(3, C, PART, (32, 32, 32), 0.1), 3000, -1.0),
    "particle2_strip_dense": (HashGridConfig(2, C, PART, (16, 16, 1), 0.05), 6000, -1.0),
    # sparse 3D with more than 64 targets per CU: the four-lane sparse density pass (smaller sparse
    # systems take sixteen lanes per target)
    "particle3_sparse_large": (HashGridConfig(3, C, PART, (32, 32, 32), 0.1), 20000, 1.2),
}


def _cloud(name, seed=3):
    g, n, radius = GRIDS[name]
    if radius < 0:  # a strip: x in [-2, 2), the other axes in [-0.3, 0.3)
        rng = np.random.default_rng(seed)
        pos = np.zeros((n, 4), np.float32)
        pos[:, 0] = rng.uniform(-2.0, 2.0, n)
        pos[:, 1:g.dim] = rng.uniform(-0.3, 0.3, (n, g.dim - 1))
        return pos, n, g
    pos = syn.uniform_ball(n, seed, radius) if g.dim == 3 else syn.uniform_disk(n, seed, radius)
    return pos, n, g


def _model16(dim, density_grad=False):
    """A 16-channel model with the rollout's usual options (state gradient, hybrid moment, log-norm),
    optionally with the density gradient: the fused kernel's FL = 5 / 13, or FL = -1."""
    if dim == 2:
        return syn.config_c1()[0].replace(density_grad=density_grad)
    return NpaConfig.growing_3dgs().replace(state_dims=16, hidden_dims=128, density_grad=density_grad)


@pytest.fixture(scope="module")
def mctx():
    c = Context(0)
    c.set_mlp_engine(_abi.MLP_MFMA)
    yield c
    c.close()


@pytest.mark.parametrize("name", list(GRIDS))
def test_hashgrid_and_neighbor_lists_bit_exact(ctx, name):
    pos, n, g = _cloud(name)
    want = O.build_hashgrid(pos, 1, n, g)
    got = K.build_hashgrid(pos, 1, n, g, ctx=ctx)
    np.testing.assert_array_equal(to_np(got.bin_offsets).astype(np.uint32), want.bin_offsets)
    np.testing.assert_array_equal(to_np(got.permutation).astype(np.uint32), want.permutation)
    np.testing.assert_array_equal(to_np(got.inverse_permutation).astype(np.uint32), want.inverse_permutation)
    off_w, idx_w = O.neighbor_lists(pos, 1, n, g)
    off_g, idx_g = K.neighbor_lists(pos, 1, n, g, ctx=ctx)
    np.testing.assert_array_equal(to_np(off_g).astype(np.uint32), off_w)
    np.testing.assert_array_equal(to_np(idx_g).astype(np.uint32), idx_w)
    assert len(idx_w) > 5 * n  # the cloud is dense enough to have neighbours across cells


def test_grid2_periodic_small_visits_wrapped_cells_more_than_once(ctx):
    """Grid mode, periodic, 6 x 5 cells: no cell is its own wrapped neighbour, but the walk of a
    3 x 3 block still crosses the domain edge; on a 2-cell axis the same cell is visited twice
    (cell_index_from_coords wraps -1 and +1 onto one cell) and its particles are listed twice."""
    g = HashGridConfig(2, P, GRID, (2, 5, 1), 0.1)
    pos = syn.uniform_disk(400, 9, 0.25)
    off_w, idx_w = O.neighbor_lists(pos, 1, 400, g)
    off_g, idx_g = K.neighbor_lists(pos, 1, 400, g, ctx=ctx)
    np.testing.assert_array_equal(to_np(off_g).astype(np.uint32), off_w)
    np.testing.assert_array_equal(to_np(idx_g).astype(np.uint32), idx_w)
    first = idx_w[off_w[0]:off_w[1]]
    assert len(first) > len(set(first.tolist()))  # a repeated neighbour


@pytest.mark.parametrize("name", ["grid3_periodic", "particle3_periodic", "grid3_clamped", "particle2_periodic"])
def test_euler_step_bit_exact(ctx, name):
    g = GRIDS[name][0]
    n, S = 2500, 16
    rng = np.random.default_rng(11)
    pos = rng.normal(scale=0.6, size=(n, 4)).astype(np.float32)
    st = (rng.normal(size=(n, S)) * 12).astype(np.float32)  # 3D: opacity logits past [-8, 24]
    dx = rng.normal(size=(n, 4)).astype(np.float32)
    ds = (rng.normal(size=(n, S)) * 10).astype(np.float32)
    mask = (rng.random(n) < 0.5).astype(np.float32)
    for m in (mask, None):
        wp, ws = O.euler_step(pos, st, dx, ds, 1, n, S, g, 0.7, m)
        gp, gs = K.euler_step(pos, st, dx, ds, 1, n, S, g, 0.7, m, ctx=ctx)
        np.testing.assert_array_equal(to_np(gp), wp)
        np.testing.assert_array_equal(to_np(gs), ws)


STEP_CASES = [(name, dg) for name in ("grid3_periodic", "particle3_periodic", "grid3_clamped",
                                      "particle2_periodic", "grid2_periodic_small", "particle2_strip_sparse",
                                      "particle3_strip_sparse", "particle2_strip_dense", "particle3_sparse_large")
              for dg in (False, True)]


def _step_case(name, density_grad):
    pos, n, g = _cloud(name)
    m = _model16(g.dim, density_grad)
    return m, g, pos, syn.normal_states(n, 16, 17), syn.seeded_weights(m, 17), n


@pytest.mark.parametrize("name,density_grad", STEP_CASES)
def test_step_bit_exact(ctx, name, density_grad):
    """One step (model.rs:768-858) and a 4-step resident rollout, bit for bit."""
    m, g, pos, st, w, n = _step_case(name, density_grad)
    mask = O.update_mask(1, n, 0.5, 0, 42)
    want = O.step(m, w, pos, st, 1, n, g, 1.0, mask)
    got = NpaModel(m, w).step(pos, st, 1, n, g, 1.0, update_mask=mask, ctx=ctx)
    np.testing.assert_array_equal(to_np(got.density), want.density)
    np.testing.assert_array_equal(to_np(got.next_positions), want.next_positions)
    np.testing.assert_array_equal(to_np(got.next_states), want.next_states)
    if g.boundary == P:  # some particles crossed the domain edge and were wrapped
        half = np.array(g.grid_size[:g.dim], np.float32) * np.float32(g.eps) * np.float32(0.5)
        assert (np.abs(pos[:, :g.dim]) >= half).any()
    want_p, want_s = O.rollout(m, w, pos, st, 1, n, g, 4, 1.0, 0.5, 42, 0)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, 1, n, g, 1.0, 0.5, 42)
    ex.step_state_many(state, 4)
    gp, gs, _ = ex.read_state(state)
    state.close()
    np.testing.assert_array_equal(to_np(gp), want_p)
    np.testing.assert_array_equal(to_np(gs), want_s)


@pytest.mark.parametrize("name,density_grad", STEP_CASES)
def test_step_mfma_engine(mctx, name, density_grad):
    m, g, pos, st, w, n = _step_case(name, density_grad)
    mask = O.update_mask(1, n, 0.5, 0, 42)
    want = O.step(m, w, pos, st, 1, n, g, 1.0, mask)
    got = NpaModel(m, w).step(pos, st, 1, n, g, 1.0, update_mask=mask, ctx=mctx)
    np.testing.assert_array_equal(to_np(got.density), want.density)
    ep, es = rel_err(got.next_positions, want.next_positions), rel_err(got.next_states, want.next_states)
    du = rel_err(to_np(got.next_states) - st, want.next_states - st)
    assert ep <= STEP_TOL and es <= STEP_TOL and du <= STEP_TOL, (ep, es, du)


def _dense_cell(dim, n_dense, n_rest, seed, boundary):
    """A cell far denser than its neighbours (as in test_gpu_parity's dense-cell perception case):
    its targets accept hundreds of neighbours over more chunks (runs of <= 64 slots) than the density
    pass records for the second pass, so the fused kernel's list overflows its LDS capacity and the
    targets past the recorded chunks test their candidates again."""
    rng = np.random.default_rng(seed)
    if dim == 2:
        g = syn.config_c1()[1].replace(boundary=boundary)
        rest = syn.uniform_disk(n_rest, seed, radius=0.4)
    else:
        g = HashGridConfig.growing_3dgs().replace(boundary=boundary)
        rest = syn.uniform_ball(n_rest, seed, radius=0.5)
    lo, hi = 0.2 * g.eps, 0.8 * g.eps  # strictly inside the cell [0, eps)^dim
    dense = np.zeros((n_dense, 4), np.float32)
    dense[:, :dim] = rng.uniform(lo, hi, size=(n_dense, dim)).astype(np.float32)
    pos = np.concatenate([dense, rest]).astype(np.float32)
    return pos[rng.permutation(len(pos))], g


DENSE_CASES = [(dim, dg, b) for dim in (2, 3) for dg, b in ((False, C), (True, C), (False, P))]


def _dense_case(dim, density_grad, boundary):
    n_dense, n_rest = (1800, 3000) if dim == 2 else (3400, 3000)
    pos, g = _dense_cell(dim, n_dense, n_rest, 5 + dim, boundary)
    n = len(pos)
    m = _model16(dim, density_grad)
    return m, g, pos, syn.normal_states(n, 16, 9), syn.seeded_weights(m, 9), n


@pytest.mark.parametrize("dim,density_grad,boundary", DENSE_CASES)
def test_dense_cell_step_bit_exact(ctx, dim, density_grad, boundary):
    m, g, pos, st, w, n = _dense_case(dim, density_grad, boundary)
    mask = O.update_mask(1, n, 0.5, 0, 42)
    want = O.step(m, w, pos, st, 1, n, g, 1.0, mask)
    got = NpaModel(m, w).step(pos, st, 1, n, g, 1.0, update_mask=mask, ctx=ctx)
    off, _ = O.neighbor_lists(pos, 1, n, g)
    assert np.diff(off.astype(np.int64)).max() > 1000  # far past the 128-entry list and the chunk records
    np.testing.assert_array_equal(to_np(got.density), want.density)
    np.testing.assert_array_equal(to_np(got.next_positions), want.next_positions)
    np.testing.assert_array_equal(to_np(got.next_states), want.next_states)


@pytest.mark.parametrize("dim,density_grad,boundary", DENSE_CASES)
def test_dense_cell_step_mfma_engine(mctx, dim, density_grad, boundary):
    m, g, pos, st, w, n = _dense_case(dim, density_grad, boundary)
    mask = O.update_mask(1, n, 0.5, 0, 42)
    want = O.step(m, w, pos, st, 1, n, g, 1.0, mask)
    got = NpaModel(m, w).step(pos, st, 1, n, g, 1.0, update_mask=mask, ctx=mctx)
    np.testing.assert_array_equal(to_np(got.density), want.density)
    ep, es = rel_err(got.next_positions, want.next_positions), rel_err(got.next_states, want.next_states)
    du = rel_err(to_np(got.next_states) - st, want.next_states - st)
    assert ep <= STEP_TOL and es <= STEP_TOL and du <= STEP_TOL, (ep, es, du)
