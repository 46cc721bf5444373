"""The HIP path against the committed golden vectors (tests/golden/c1_small.npz), through the
C ABI: hashgrid, neighbour lists and mask bit-exact; perception and one step within 1e-5; the
16-step rollout within 1e-3; the splat of the rolled-out state at >= 100 dB PSNR."""
import numpy as np
import pytest

from burn_automata_amd import kernels as K
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from tests.golden import make_golden as G
from tests.helpers import psnr, rel_err, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def case():
    return G.inputs(), G.load()


def test_golden_hashgrid_and_neighbours(ctx, case):
    (model, grid, pos, st, w, _), gold = case
    g = K.build_hashgrid(pos, 1, G.N, grid, ctx=ctx)
    np.testing.assert_array_equal(to_np(g.bin_offsets).astype(np.uint32), gold["bin_offsets"])
    np.testing.assert_array_equal(to_np(g.permutation).astype(np.uint32), gold["permutation"])
    np.testing.assert_array_equal(to_np(g.inverse_permutation).astype(np.uint32),
                                  gold["inverse_permutation"])
    off, idx = K.neighbor_lists(pos, 1, G.N, grid, ctx=ctx)
    np.testing.assert_array_equal(to_np(off).astype(np.uint32), gold["neighbor_offsets"])
    np.testing.assert_array_equal(to_np(idx).astype(np.uint32), gold["neighbor_indices"])


def test_golden_perception_mask_and_step(ctx, case):
    (model, grid, pos, st, w, _), gold = case
    per = K.perceive_with_options(pos, st, 1, G.N, model.state_dims, grid,
                                  model.perception_options(), ctx=ctx)
    assert rel_err(per.density, gold["density"]) <= 1e-5
    assert rel_err(per.features, gold["features"]) <= 1e-5
    mask = K.update_mask(1, G.N, 0.5, 0, G.SEED, ctx=ctx)
    np.testing.assert_array_equal(to_np(mask), gold["mask"])
    out = NpaModel(model, w).step(pos, st, 1, G.N, grid, 1.0, update_mask=mask, ctx=ctx)
    assert rel_err(out.next_positions, gold["step_positions"]) <= 1e-5
    assert rel_err(out.next_states, gold["step_states"]) <= 1e-5


def test_golden_rollout_and_splat(ctx, case):
    (model, grid, pos, st, w, splat), gold = case
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(model, w), pos, st, 1, G.N, grid, 1.0, 0.5, G.SEED)
    ex.step_state_many(state, G.ROLLOUT_STEPS)
    gp, gs, _ = ex.read_state(state)
    ep, es = rel_err(gp, gold["rollout_positions"]), rel_err(gs, gold["rollout_states"])
    print(f"golden {G.ROLLOUT_STEPS}-step rollout rel err pos={ep:.3e} state={es:.3e}")
    assert ep <= 1e-3 and es <= 1e-3
    img = ex.splat_2d(state, splat)
    assert psnr(img, gold["splat"]) >= 100.0
    state.close()
