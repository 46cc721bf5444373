"""The committed golden vectors (tests/golden/c1_small.npz) against the seeded generator and the
oracle: the inputs still hash to the recorded digest and the oracle still reproduces every output
bit for bit. A deliberate change of the oracle regenerates the file with
tests/golden/make_golden.py; an accidental one fails here."""
import numpy as np
import pytest

from tests.golden import make_golden as G


@pytest.fixture(scope="module")
def golden():
    return G.load()


def test_inputs_match_recorded_digest(golden):
    model, grid, pos, st, w, _ = G.inputs()
    assert G.digest(pos, st, w["w1"], w["b1"], w["w2"], w["b2"]) == str(golden["input_digest"])


def test_oracle_reproduces_golden_outputs(golden):
    fresh = G.compute()
    for key, want in golden.items():
        if key == "input_digest":
            continue
        np.testing.assert_array_equal(fresh[key], want, err_msg=key)


def test_golden_case_is_not_degenerate(golden):
    per_particle = np.diff(golden["neighbor_offsets"].astype(np.int64))
    assert per_particle.min() >= 1 and per_particle.mean() > 5  # self plus real neighbourhoods
    assert 0.3 < golden["mask"].mean() < 0.7
    moved = np.abs(golden["rollout_positions"] - G.inputs()[2]).max()
    assert moved > 1e-3 and np.all(np.isfinite(golden["rollout_states"]))
