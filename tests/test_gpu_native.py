"""A non-Python caller: tests/native/c_step.c, compiled against include/npa_abi.h and linked to
libnpa_hip.so, runs one host-I/O npa_step and a 4-step resident rollout (npa_state_*) of a C1
system from raw float32 files; its outputs must equal the oracle's NpaModel::step_cpu
(crates/burn_automata/src/model.rs:768-858) and rollout (rollout/mod.rs:240-297) bit for bit."""
import os
import subprocess

import numpy as np
import pytest

from burn_automata_amd import synthetic as syn
from oracle import oracle as O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "native", "c_step")


def test_c_caller_step_and_rollout(tmp_path):
    if not os.path.exists(EXE):
        from tests.native import build_c_step
        build_c_step.build()
    w = syn.workload("c1", particles=2048)
    m, n = w["model"], w["n"]
    S, H = m.state_dims, m.hidden_dims
    assert m.perception_dims() == 4 * S and m.update_dims() == 2 + S
    mask = O.update_mask(1, n, 0.5, 0, 42)
    wt = w["weights"]
    for name, arr in (("positions", w["positions"]), ("states", w["states"]), ("w1", wt["w1"]), ("b1", wt["b1"]),
                      ("w2", wt["w2"]), ("b2", wt["b2"]), ("mask", mask)):
        np.ascontiguousarray(arr, np.float32).tofile(tmp_path / f"{name}.f32")
    steps = 4
    r = subprocess.run([EXE, str(tmp_path), str(n), str(S), str(H), str(steps)], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr

    def load(name, shape):
        return np.fromfile(tmp_path / f"{name}.f32", np.float32).reshape(shape)

    want = O.step(m, wt, w["positions"], w["states"], 1, n, w["grid"], 1.0, mask)
    np.testing.assert_array_equal(load("step_positions", (n, 4)), want.next_positions)
    np.testing.assert_array_equal(load("step_states", (n, S)), want.next_states)
    np.testing.assert_array_equal(load("step_density", (n,)), want.density)
    wp, ws = O.rollout(m, wt, w["positions"], w["states"], 1, n, w["grid"], steps, 1.0, 0.5, 42, 0)
    np.testing.assert_array_equal(load("roll_positions", (n, 4)), wp)
    np.testing.assert_array_equal(load("roll_states", (n, S)), ws)


def test_mfma_product_equals_vector_multiply():
    """The fused update kernel's bit-exact engine takes layer-1 products from v_mfma_f32_4x4x1f32
    with a -0.0 accumulator: each must be v_mul_f32's rounded product bit for bit (ordinary values,
    zeros of both signs, denormal inputs and products; tests/native/mfma_product.cpp)."""
    exe = os.path.join(HERE, "native", "mfma_product")
    if not os.path.exists(exe):
        from tests.native import build_c_step
        build_c_step.build_mfma_product()
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "mismatches 0 of" in r.stdout, r.stdout + r.stderr
