"""Writes tests/golden/c1_small.npz: a 256-particle C1-style system and the oracle's outputs for it.

Inputs come from the product's seeded generator (burn_automata_amd.synthetic) and are rebuilt by
the tests; the file holds their SHA-256 digests (so a change of the generator is caught) and the
oracle's outputs: hashgrid, neighbour lists, perception, one masked step, a 16-step rollout and a
64x64 splat of the final state. tests/test_golden.py checks that the oracle still reproduces them;
tests/test_gpu_golden.py checks the HIP path against them.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PATH = os.path.join(HERE, "c1_small.npz")
N = 256
ROLLOUT_STEPS = 16
SEED = 42


def inputs():
    """C1 model/grid (S=16, H=128, eps = eps0 = 0.05, Particle 64x64) on 256 particles in a disk
    of radius 0.25, so each particle has about as many neighbours as in C1."""
    from burn_automata_amd import synthetic as syn
    from burn_automata_amd.config import Splat2dConfig

    model, grid = syn.config_c1(N, SEED)
    pos = syn.uniform_disk(N, SEED, radius=0.25)
    st = syn.normal_states(N, model.state_dims, SEED)
    w = syn.seeded_weights(model, SEED)
    splat = Splat2dConfig(image_size=64, sigma=1.0, pixel_size=2.0 / 64, lo=-0.5, hi=0.5)
    return model, grid, pos, st, w, splat


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def compute():
    from oracle import oracle as O

    model, grid, pos, st, w, splat = inputs()
    g = O.build_hashgrid(pos, 1, N, grid)
    noff, nidx = O.neighbor_lists(pos, 1, N, grid)
    per = O.perceive_with_options(pos, st, 1, N, model.state_dims, grid, model.perception_options())
    mask = O.update_mask(1, N, 0.5, 0, SEED)
    out = O.step(model, w, pos, st, 1, N, grid, 1.0, mask)
    rp, rs = O.rollout(model, w, pos, st, 1, N, grid, ROLLOUT_STEPS, 1.0, 0.5, SEED, 0)
    img = O.splat_particles_2d(rp, O.tail_colors(rs, model.state_dims), splat)
    return dict(
        input_digest=np.array(digest(pos, st, w["w1"], w["b1"], w["w2"], w["b2"])),
        bin_offsets=g.bin_offsets, permutation=g.permutation,
        inverse_permutation=g.inverse_permutation, neighbor_offsets=noff, neighbor_indices=nidx,
        density=per.density, blurred_state=per.blurred_state, features=per.features, mask=mask,
        step_positions=out.next_positions, step_states=out.next_states, rollout_positions=rp,
        rollout_states=rs, splat=img)


def load():
    with np.load(PATH, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


if __name__ == "__main__":
    np.savez_compressed(PATH, **compute())
    print(f"wrote {PATH} ({os.path.getsize(PATH)} bytes)")
