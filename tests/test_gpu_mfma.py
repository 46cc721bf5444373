"""The update MLP on the fp32 matrix cores (NPA_MLP_MFMA) against the CPU oracle (runs on an MI355X).

The matrix cores accumulate the products in their own order, so the step is compared within the
single-step gate (1e-5, norm-relative) instead of bit for bit; everything before the MLP (the
hashgrid, density and features) is unchanged, so the density stays bit-exact.
"""
import numpy as np
import pytest

from burn_automata_amd import _abi
from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import HashGridConfig, NpaConfig
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from burn_automata_amd.runtime import Context
from oracle import oracle as O
from tests.helpers import rel_err, to_np

pytestmark = pytest.mark.gpu

STEP_TOL = 1e-5


@pytest.fixture(scope="module")
def mctx():
    c = Context(0)
    c.set_mlp_engine(_abi.MLP_MFMA)
    yield c
    c.close()


def _case(name):
    if name in ("c1", "c2", "c5"):
        w = syn.workload(name)
        return w["model"], w["grid"], w["positions"], w["states"], w["weights"], w["batch"], w["n"]
    if name == "growing_3d":
        m, g, n = NpaConfig.growing_3dgs(), HashGridConfig.growing_3dgs(), 2048
        return (m, g, syn.uniform_ball(n, 4, 0.5), syn.normal_states(n, m.state_dims, 4),
                syn.seeded_weights(m, 4), 1, n)
    if name == "c4":
        w = syn.workload("c4", particles=4096)
        return w["model"], w["grid"], w["positions"], w["states"], w["weights"], 1, w["n"]
    raise KeyError(name)


@pytest.mark.parametrize("name", ["c1", "c2", "c5", "growing_3d", "c4"])
def test_mfma_step_within_single_step_gate(mctx, name):
    m, g, pos, st, w, b, n = _case(name)
    mask = O.update_mask(b, n, 0.5, 0, 42)
    want = O.step(m, w, pos, st, b, n, g, 1.0, mask)
    got = NpaModel(m, w).step(pos, st, b, n, g, 1.0, update_mask=mask, ctx=mctx)
    np.testing.assert_array_equal(to_np(got.density), want.density)
    ep, es = rel_err(got.next_positions, want.next_positions), rel_err(got.next_states, want.next_states)
    # the update itself (next - current) carries the MLP's rounding; compare it on its own scale too
    du = rel_err(to_np(got.next_states) - st, want.next_states - st)
    print(f"{name}: mfma step rel err pos={ep:.2e} state={es:.2e} update={du:.2e}")
    assert ep <= STEP_TOL and es <= STEP_TOL and du <= STEP_TOL
    off = mask == 0  # masked-out particles take no update on either engine
    np.testing.assert_array_equal(to_np(got.next_states)[off], want.next_states[off])


@pytest.fixture(scope="module")
def bctx():
    c = Context(0)
    c.set_mlp_engine(_abi.MLP_MFMA_BF16)
    yield c
    c.close()


def _bf16_valued(weights):
    """Each weight rounded to bf16 (nearest even), as f32: the weights the bf16 engine takes exactly."""
    out = {}
    for k, v in weights.items():
        u = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        out[k] = r.astype(np.uint32).view(np.float32).reshape(np.shape(v))
    return out


@pytest.mark.parametrize("name", ["c5", "c1", "c2", "growing_3d"])
def test_bf16_engine_step_within_single_step_gate(bctx, name):
    """NPA_MLP_MFMA_BF16: layer 1 on v_mfma_f32_4x4x4bf16_1k with bf16x3 features. With bf16-valued
    weights (C5's are; the others are rounded to bf16 here) every product is exact, so the step
    stays within the single-step gate; 3D systems run the fp32 matrix-core engine."""
    m, g, pos, st, w, b, n = _case(name)
    if name != "c5":
        w = _bf16_valued(w)
    mask = O.update_mask(b, n, 0.5, 0, 42)
    want = O.step(m, w, pos, st, b, n, g, 1.0, mask)
    got = NpaModel(m, w).step(pos, st, b, n, g, 1.0, update_mask=mask, ctx=bctx)
    np.testing.assert_array_equal(to_np(got.density), want.density)
    ep, es = rel_err(got.next_positions, want.next_positions), rel_err(got.next_states, want.next_states)
    du = rel_err(to_np(got.next_states) - st, want.next_states - st)
    print(f"{name}: bf16 engine step rel err pos={ep:.2e} state={es:.2e} update={du:.2e}")
    assert ep <= STEP_TOL and es <= STEP_TOL and du <= STEP_TOL
    off = mask == 0
    np.testing.assert_array_equal(to_np(got.next_states)[off], want.next_states[off])


def test_mfma_state_engine_and_errors(ctx):
    m, g, pos, st, w, b, n = _case("c1")
    ex = HipAutomataExecutor(ctx=ctx)
    s_valu = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, 0.5, 42)
    s_mfma = ex.create_state(NpaModel(m, w), pos, st, b, n, g, 1.0, 0.5, 42)
    s_mfma.set_mlp_engine(_abi.MLP_MFMA)
    ex.step_state(s_valu)
    ex.step_state(s_mfma)
    pv, sv, _ = ex.read_state(s_valu)
    pm, sm, _ = ex.read_state(s_mfma)
    assert rel_err(sm, sv) <= STEP_TOL and rel_err(pm, pv) <= STEP_TOL
    with pytest.raises(_abi.InvalidArgument):
        s_mfma.set_mlp_engine(7)
    s_valu.close()
    s_mfma.close()



@pytest.mark.parametrize("name,systems", [("c1", 1), ("c2", 1), ("c5", 8)])
def test_mfma_rollout_drift_is_the_dynamics_own(ctx, name, systems):
    """64 resident steps on the matrix-core engine. The rollout is chaotic: the reference itself,
    started from states one ulp away, ends about as far from its own unperturbed rollout as any
    engine whose roundings differ (the bit-exact VALU engine is the only one inside the 1e-3
    64-step gate). So the matrix-core rollout is pinned to the reference's sensitivity: its
    64-step distance from the oracle is at most 10x the oracle's distance from itself after a
    one-ulp perturbation of the initial states. C5 runs 8 of its 64 systems (bf16-representable
    weights, as the workload specifies) so that the oracle finishes in seconds."""
    w = syn.workload(name)
    m, g, n = w["model"], w["grid"], w["n"]
    b = systems
    pos, st = w["positions"][:b * n], w["states"][:b * n]
    steps = 64
    want_p, want_s = O.rollout(m, w["weights"], pos, st, b, n, g, steps, 1.0, 0.5, 42, 0)
    st_ulp = np.nextafter(st, np.float32(np.inf)).astype(np.float32)
    ulp_p, ulp_s = O.rollout(m, w["weights"], pos, st_ulp, b, n, g, steps, 1.0, 0.5, 42, 0)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w["weights"]), pos, st, b, n, g, 1.0, 0.5, 42)
    try:
        state.set_mlp_engine(_abi.MLP_MFMA)
        ex.step_state_many(state, steps)
        gp, gs, _ = ex.read_state(state)
    finally:
        state.close()
    ep, es = rel_err(gp, want_p), rel_err(gs, want_s)
    rp, rs = rel_err(ulp_p, want_p), rel_err(ulp_s, want_s)
    print(f"{name} x{b}: 64 steps, mfma vs oracle pos={ep:.3e} state={es:.3e}; "
          f"oracle one-ulp perturbation pos={rp:.3e} state={rs:.3e}")
    assert np.isfinite(to_np(gp)).all() and np.isfinite(to_np(gs)).all()
    assert ep <= 10 * rp and es <= 10 * rs

