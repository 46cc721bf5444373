"""Independent contexts used from separate host threads at the same time (runs on an MI355X).

The C ABI is thread-safe for distinct contexts and streams (the kernels' one-time launch set-up is
per device and guarded; everything else lives in the context or the state). Two threads, each with
its own context on its own stream, run a fused step and a resident rollout concurrently — a 2D
system on one, a 3D system on the other — and each result must equal the CPU oracle bit for bit.
"""
import threading

import numpy as np
import pytest

from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import HashGridConfig, NpaConfig
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from burn_automata_amd.runtime import Context
from oracle import oracle as O
from tests.helpers import to_np

pytestmark = pytest.mark.gpu


def _systems():
    m2, g2 = syn.config_c1()
    n2 = 4096
    m3 = NpaConfig.growing_3dgs().replace(state_dims=16, hidden_dims=128)
    g3 = HashGridConfig.growing_3dgs()
    n3 = 3000
    return [
        (m2, g2, syn.uniform_disk(n2, 81), syn.normal_states(n2, 16, 81), syn.seeded_weights(m2, 81), n2),
        (m3, g3, syn.uniform_ball(n3, 82, 0.5), syn.normal_states(n3, 16, 82), syn.seeded_weights(m3, 82), n3),
    ]


def test_two_contexts_on_two_threads():
    import torch

    systems = _systems()
    steps = 12
    want = []
    for m, g, pos, st, w, n in systems:
        mask = O.update_mask(1, n, 0.5, 5, 42)
        one = O.step(m, w, pos, st, 1, n, g, 1.0, mask)
        rp, rs = O.rollout(m, w, pos, st, 1, n, g, steps, 1.0, 0.5, 42, 0)
        want.append((mask, one, rp, rs))
    results = [None, None]
    errors = []
    start = threading.Barrier(2)

    def worker(k):
        try:
            m, g, pos, st, w, n = systems[k]
            mask = want[k][0]
            stream = torch.cuda.Stream(device=0)  # default priority
            # torch's current stream is the context's: the wrapper's tensors are allocated, copied and
            # freed in the same stream order as the library's kernels
            with torch.cuda.stream(stream):
                ctx = Context(0)
                model = NpaModel(m, w)
                ex = HipAutomataExecutor(ctx=ctx)
                start.wait()
                out = model.step(pos, st, 1, n, g, 1.0, update_mask=mask, ctx=ctx)
                state = ex.create_state(model, pos, st, 1, n, g, 1.0, 0.5, 42)
                for _ in range(3):
                    ex.step_state_many(state, steps // 3)
                gp, gs, _ = ex.read_state(state)
                ctx.synchronize()
                results[k] = (to_np(out.next_positions).copy(), to_np(out.next_states).copy(),
                              to_np(gp).copy(), to_np(gs).copy())
                state.close()
                ctx.close()
        except BaseException as e:  # reported by the main thread
            errors.append((k, repr(e)))
            start.abort()

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for k in range(2):
        mask, one, rp, rs = want[k]
        np_, ns, gp, gs = results[k]
        np.testing.assert_array_equal(np_, one.next_positions)
        np.testing.assert_array_equal(ns, one.next_states)
        np.testing.assert_array_equal(gp, rp)
        np.testing.assert_array_equal(gs, rs)
