"""BASELINE.json's workloads C3-C5 on the HIP path, against the CPU oracle (runs on an MI355X).

C3  1,048,576 particles from an 8-component Gaussian mixture (max/mean cell count above 50):
    the full-size hashgrid bit for bit; one full-size step checked at sampled particles (their
    density from the oracle's density pass, their next state from the oracle's step evaluated
    with the device's densities); the same mixture at 65,536 particles checked whole.
C4  16,384 particles on a closed 3D surface, F=80, O=19: step and 64-step rollout, then the
    oriented Gaussian decode and its 512x512 EWA raster (the bench's decode), the device's frame
    against the oracle's raster of the oracle's decode.
C5  64 systems x 4,096 particles with bf16-rounded weights: step and rollout, then every system
    splatted into its own 128x128 window of a 1024x1024 image.
"""
import numpy as np
import pytest

from burn_automata_amd import kernels as K
from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import RasterColor
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from oracle import oracle as O
from tests.helpers import psnr, rel_err, to_np

pytestmark = pytest.mark.gpu

ROLLOUT_TOL = 1e-3


def _rollout_pair(ctx, w, steps):
    b, n = w["batch"], w["n"]
    want_p, want_s = O.rollout(w["model"], w["weights"], w["positions"], w["states"], b, n,
                               w["grid"], steps, w["dt"], w["update_prob"], w["seed"], 0)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(w["model"], w["weights"]), w["positions"], w["states"], b, n,
                            w["grid"], w["dt"], w["update_prob"], w["seed"])
    ex.step_state_many(state, steps)
    return ex, state, want_p, want_s


def test_c3_full_size_hashgrid_bit_exact(ctx):
    w = syn.workload("c3")
    n = w["n"]
    want = O.build_hashgrid(w["positions"], 1, n, w["grid"])
    got = K.build_hashgrid(w["positions"], 1, n, w["grid"], ctx=ctx)
    np.testing.assert_array_equal(to_np(got.bin_offsets).astype(np.uint32), want.bin_offsets)
    np.testing.assert_array_equal(to_np(got.permutation).astype(np.uint32), want.permutation)
    np.testing.assert_array_equal(to_np(got.inverse_permutation).astype(np.uint32),
                                  want.inverse_permutation)
    counts = np.diff(want.bin_offsets.astype(np.int64))
    assert counts.max() / counts.mean() > 50  # the workload's stated skew


def test_c3_full_size_step_at_sampled_particles(ctx):
    w = syn.workload("c3")
    m, g, n = w["model"], w["grid"], w["n"]
    pos, st = w["positions"], w["states"]
    mask = O.update_mask(1, n, 0.5, 0, w["seed"])
    got = NpaModel(m, w["weights"]).step(pos, st, 1, n, g, 1.0, update_mask=mask, ctx=ctx)
    dens = to_np(got.density)
    gp, gs = to_np(got.next_positions), to_np(got.next_states)
    assert np.isfinite(dens).all() and np.isfinite(gp).all() and np.isfinite(gs).all()
    # particles with update mask 0 keep their values (2D clamped grid: no wrap, no clamp)
    off = mask == 0
    np.testing.assert_array_equal(gp[off], pos[off])
    np.testing.assert_array_equal(gs[off], st[off])
    # samples: half from the 16 most crowded bins, half uniform
    snap = O.build_hashgrid(pos, 1, n, g)
    bo = snap.bin_offsets.astype(np.int64)
    rng = np.random.default_rng(3)
    hot = np.argsort(np.diff(bo))[-16:]
    hot_slots = np.concatenate([np.arange(bo[h], bo[h + 1]) for h in hot])
    hot_ids = snap.permutation[rng.choice(hot_slots, 384, replace=False)]
    sel = np.unique(np.concatenate([hot_ids, rng.choice(n, 384, replace=False)])).astype(np.uint32)
    want_d = O.density_rows(pos, 1, n, g, sel)
    np.testing.assert_array_equal(dens[sel], want_d)
    tgt = sel[mask[sel] != 0]
    wp, ws = O.step_rows(m, w["weights"], pos, st, 1, n, g, 1.0, mask, dens, tgt)
    np.testing.assert_array_equal(gp[tgt], wp)
    np.testing.assert_array_equal(gs[tgt], ws)


def test_c3_mixture_at_65536_step_bit_exact(ctx):
    w = syn.workload("c3", particles=65536)
    m, g, n = w["model"], w["grid"], w["n"]
    mask = O.update_mask(1, n, 0.5, 0, w["seed"])
    want = O.step(m, w["weights"], w["positions"], w["states"], 1, n, g, 1.0, mask)
    got = NpaModel(m, w["weights"]).step(w["positions"], w["states"], 1, n, g, 1.0,
                                         update_mask=mask, ctx=ctx)
    np.testing.assert_array_equal(to_np(got.density), want.density)
    np.testing.assert_array_equal(to_np(got.next_positions), want.next_positions)
    np.testing.assert_array_equal(to_np(got.next_states), want.next_states)


def test_c4_surface_rollout_decode_and_raster(ctx):
    w = syn.workload("c4")
    assert w["model"].perception_dims() == 80 and w["model"].update_dims() == 19
    steps = 64
    ex, state, want_p, want_s = _rollout_pair(ctx, w, steps)
    gp, gs, _ = ex.read_state(state)
    ep, es = rel_err(gp, want_p), rel_err(gs, want_s)
    print(f"c4: {steps}-step rollout rel err pos={ep:.3e} state={es:.3e}")
    assert ep <= ROLLOUT_TOL and es <= ROLLOUT_TOL
    np.testing.assert_array_equal(to_np(gp), want_p)
    np.testing.assert_array_equal(to_np(gs), want_s)
    dec = ex.decode_gaussians_3d(state, w["decode"])
    want_dec = O.decode_gaussians_3d(want_p, want_s, w["model"].state_dims, w["decode"])
    for k in want_dec:
        assert rel_err(dec[k], want_dec[k]) <= 1e-6, k
    # the workload's decode: the oriented Gaussians drawn by the EWA raster from the workload's
    # camera (decode_gaussians_3d's colours as RGB), in one call on the resident state
    cam = w["camera"]
    img = to_np(ex.raster_gaussians_3d(state, w["decode"], cam))
    want_img = O.raster_gaussians_3d(want_dec["position_visibility"], want_dec["spherical_harmonic"],
                                     want_dec["rotation"], want_dec["scale_opacity"],
                                     cam.replace(color_mode=RasterColor.Rgb, sh_degree=0))
    assert img.shape == (512, 512, 4)
    d = np.abs(img.astype(np.float64) - want_img)
    p = psnr(img, want_img)
    off = float((d > 1e-4).mean())
    lit = float((want_img[..., 3] > 0.01).mean())
    print(f"c4: decoded 512x512 EWA raster psnr={p:.1f} dB, values off by >1e-4 {off:.2e}, lit {lit:.2f}")
    # the raster's bar (tests/test_gpu_raster.py): an ulp of exp may move a pixel across the 1/255
    # alpha floor or the 1e-4 transmittance cut
    assert p >= 90.0 and off <= 1e-4
    assert lit > 0.05  # the surface is in view
    state.close()


def test_c5_batched_bf16_rollout_and_tiled_splat(ctx):
    w = syn.workload("c5")
    b, n = w["batch"], w["n"]
    assert b == 64 and np.array_equal(syn.round_bf16(w["weights"]["w1"]), w["weights"]["w1"])
    mask = O.update_mask(b, n, 0.5, 0, w["seed"])
    want = O.step(w["model"], w["weights"], w["positions"], w["states"], b, n, w["grid"], 1.0, mask)
    got = NpaModel(w["model"], w["weights"]).step(w["positions"], w["states"], b, n, w["grid"],
                                                  1.0, update_mask=mask, ctx=ctx)
    np.testing.assert_array_equal(to_np(got.next_positions), want.next_positions)
    np.testing.assert_array_equal(to_np(got.next_states), want.next_states)
    steps = 16
    ex, state, want_p, want_s = _rollout_pair(ctx, w, steps)
    gp, gs, _ = ex.read_state(state)
    ep, es = rel_err(gp, want_p), rel_err(gs, want_s)
    print(f"c5: {steps}-step rollout rel err pos={ep:.3e} state={es:.3e}")
    assert ep <= ROLLOUT_TOL and es <= ROLLOUT_TOL
    np.testing.assert_array_equal(to_np(gp), want_p)
    np.testing.assert_array_equal(to_np(gs), want_s)
    cfg, tx = w["splat"], w["tiles_x"]
    img = to_np(ex.splat_2d_tiled(state, cfg, tx))
    size = cfg.image_size
    assert img.shape == (b // tx * size, tx * size, 4)
    colors = O.tail_colors(want_s, w["model"].state_dims)
    want_img = np.zeros_like(img)
    for k in range(b):
        r, c = divmod(k, tx)
        tile = O.splat_particles_2d(want_p[k * n:(k + 1) * n], colors[k * n:(k + 1) * n], cfg)
        want_img[r * size:(r + 1) * size, c * size:(c + 1) * size] = tile.reshape(size, size, 4)
    p = psnr(img, want_img)
    print(f"c5: tiled 1024x1024 image psnr={p:.1f} dB")
    assert p >= 100.0
    state.close()


def test_tiled_splat_matches_separate_splats(ctx):
    """A partial last row of windows stays zero; each window equals its system's own splat."""
    b, n, tx = 5, 700, 3
    pos = np.concatenate([syn.uniform_disk(n, 30 + k, radius=1.05) for k in range(b)])
    colors = O.tail_colors(syn.normal_states(b * n, 16, 30, std=0.3), 16)
    from burn_automata_amd.config import Splat2dConfig
    cfg = Splat2dConfig(image_size=40, sigma=1.5, pixel_size=2.0 / 40)
    img = to_np(K.splat_particles_2d_tiled(pos, colors, b, n, cfg, tx, ctx=ctx))
    assert img.shape == (2 * 40, 3 * 40, 4)
    for k in range(6):
        r, c = divmod(k, tx)
        win = img[r * 40:(r + 1) * 40, c * 40:(c + 1) * 40].reshape(-1, 4)
        if k >= b:
            assert not win.any()
            continue
        alone = to_np(K.splat_particles_2d(pos[k * n:(k + 1) * n], colors[k * n:(k + 1) * n], cfg,
                                           ctx=ctx))
        np.testing.assert_array_equal(win, alone)


def test_bpk_model_drives_the_rollout(ctx):
    """A model read from a .bpk container (burn_automata_amd.bpk, import.rs:378-498) steps on the
    device exactly as the oracle steps the weights it was written from."""
    from burn_automata_amd import bpk
    from tests.test_bpk import container, manifest_json

    w = syn.workload("c1", particles=2048)
    pos = w["positions"]
    st = w["states"]
    man = bpk.load_manifest_bytes(container(manifest_json(w["model"], w["grid"], w["weights"],
                                                          initialization=(pos, st))))
    model = man.into_model()
    p0, s0 = man.initialization
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(model, p0, s0, 1, p0.shape[0], man.hashgrid, 1.0, 0.5, 42)
    ex.step_state_many(state, 8)
    gp, gs, _ = ex.read_state(state)
    want_p, want_s = O.rollout(man.config, man.weights, p0, s0, 1, p0.shape[0], man.hashgrid, 8, 1.0,
                               0.5, 42, 0)
    np.testing.assert_array_equal(to_np(gp), want_p)
    np.testing.assert_array_equal(to_np(gs), want_s)
    state.close()
