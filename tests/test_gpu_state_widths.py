"""State rows of every width the payload scatters load whole (runs on an MI355X).

The small-system and binned hashgrid builds load a particle's state row with its position, as
1, 2, 4, 6 or 8 float4s when the row is a whole number of them (S = 4, 8, 16, 24, 32), and write
a particle outside the step's update mask to the step's output from those registers; any other
width takes the element-wise copy. These cases drive the widths the configs do not (S = 4 and
S = 32 on the two-launch build, S = 8 and S = 32 on the binned 3D build, S = 5 element-wise)
through perception (sorted state rows: features and density against the oracle) and through
rollouts (held particles: bit-exact against the oracle's steps, step.rs:4-55)."""
import numpy as np
import pytest

from burn_automata_amd import kernels as K
from burn_automata_amd.config import HashGridConfig, NpaConfig
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from burn_automata_amd import synthetic as syn
from oracle import oracle as O
from tests.helpers import rel_err, to_np

pytestmark = pytest.mark.gpu

STEP_TOL = 1e-5


def _case(name):
    """(model, grid, positions, states, particles): 2D on C1's grid (4,096 bins, the two-launch
    build) or 3D on growing_3dgs' 32^3 Particle grid (the binned build)."""
    c1_model, c1_grid = syn.config_c1()
    S = int(name.split("_s")[1])
    if name.startswith("sys"):
        n = 2000
        return c1_model.replace(state_dims=S), c1_grid, syn.uniform_disk(n, 90 + S), syn.normal_states(n, S, 90 + S), n
    n = 3000
    m = NpaConfig.growing_3dgs().replace(state_dims=S, hidden_dims=64)
    return m, HashGridConfig.growing_3dgs(), syn.uniform_ball(n, 70 + S, radius=0.6), \
        syn.normal_states(n, S, 70 + S, std=1.0), n


CASES = ["sys_s4", "sys_s32", "sys_s5", "bins_s8", "bins_s32"]


@pytest.mark.parametrize("name", CASES)
def test_perceive_state_width(ctx, name):
    m, g, pos, st, n = _case(name)
    S, opts = m.state_dims, m.perception_options()
    want = O.perceive_with_options(pos, st, 1, n, S, g, opts)
    got = K.perceive_with_options(pos, st, 1, n, S, g, opts, ctx=ctx)
    assert got.feature_dims == want.feature_dims
    np.testing.assert_array_equal(to_np(got.density), want.density)
    for field in ("features", "blurred_state", "state_gradient", "density_gradient"):
        e = rel_err(getattr(got, field), getattr(want, field))
        assert e <= STEP_TOL, f"{field}: {e}"


@pytest.mark.parametrize("name", CASES)
def test_rollout_state_width(ctx, name):
    m, g, pos, st, n = _case(name)
    w = syn.seeded_weights(m, 11)
    steps = 8
    want_p, want_s = O.rollout(m, w, pos, st, 1, n, g, steps, 1.0, 0.5, 42, 0)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, 1, n, g, 1.0, 0.5, 42)
    try:
        ex.step_state_many(state, steps)
        gp, gs, _ = ex.read_state(state)
    finally:
        state.close()
    # the VALU engine sums in the reference's order and the held particles are copied (wrapped,
    # clamped) exactly: the rollout is the oracle's bit for bit
    np.testing.assert_array_equal(to_np(gp), want_p)
    np.testing.assert_array_equal(to_np(gs), want_s)
