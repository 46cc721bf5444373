"""The projected 3D render (render_loss raster) on the HIP path, against the CPU oracle.

npa_render_views replaces project_positions + splat_projected
(crates/burn_automata/src/render_loss/projection.rs:11-29, render_loss/image.rs:18-79) for several
views in one pipeline; npa_render_attributes replaces state_tail_render_attributes
(render_loss/attributes.rs:15-87); npa_state_render_views draws the particle images of
mesh_multiview_render_loss_from_trace (render_loss.rs:107-141) from a device-resident state.

Tolerances: the device evaluates the splat weight as 2^(-d^2 log2(e) / 2 sigma^2) with one
combined scale, splits each footprint's weight sum over 16 lanes and each tile's particle list
into chunks of 256 summed in order; all of this changes rounding only, so max |GPU - CPU| <= 1e-5
of the image's peak and PSNR >= 100 dB (measured: <= 3e-6, >= 139 dB). Attributes: 1e-6 (expf).
"""
import numpy as np
import pytest

from burn_automata_amd import _abi
from burn_automata_amd import kernels as K
from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import ALL_VIEWS, GaussianDecodeMode, RenderLossConfig, RenderViewPreset
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from oracle import oracle as O
from tests.helpers import psnr, rel_err, to_np

pytestmark = pytest.mark.gpu

IMG_TOL = 1e-5
ATTR_TOL = 1e-6


def _particles(n, seed, spread=1.6):
    rng = np.random.default_rng(seed)
    pos = np.zeros((n, 4), np.float32)
    pos[:, :3] = rng.uniform(-spread, spread, (n, 3))
    pos[:, 3] = rng.uniform(-1, 1, n)
    col = rng.uniform(0, 1, (n, 3)).astype(np.float32)
    op = rng.uniform(-0.2, 1.2, n).astype(np.float32)    # both clamps of image.rs:68
    sg = rng.uniform(0.2, 7.0, n).astype(np.float32)     # both sigma clamps of image.rs:39
    return pos, col, op, sg


def _check_images(got, want, what):
    got = to_np(got).reshape(want.shape)
    e, p = rel_err(got, want), psnr(got, want)
    print(f"{what}: rel err {e:.3e} psnr {p:.1f} dB")
    assert e <= IMG_TOL and p >= 100.0, what


@pytest.mark.parametrize("size,n", [(64, 3000), (100, 2500), (1, 50), (257, 20000)])
def test_render_views_match_the_oracle(ctx, size, n):
    pos, col, op, sg = _particles(n, size)
    cfg = RenderLossConfig(image_size=size)
    want = O.render_views(pos, col, op, sg, ALL_VIEWS, cfg)
    got = K.render_views(pos, col, op, sg, cfg, ALL_VIEWS, ctx=ctx)
    assert got.shape == (4, size, size, 5)
    _check_images(got, want, f"render {size}x{size} n={n}")
    again = K.render_views(pos, col, op, sg, cfg, ALL_VIEWS, ctx=ctx)
    np.testing.assert_array_equal(to_np(again), to_np(got))  # deterministic


def test_render_views_order_repeats_and_empty_input(ctx):
    pos, col, op, sg = _particles(800, 7, spread=1.0)
    cfg = RenderLossConfig(image_size=48, sigma=3.0, min_sigma=0.5, max_sigma=6.0, world_scale=1.1)
    views = (RenderViewPreset.Iso, RenderViewPreset.Xy, RenderViewPreset.Iso)
    got = to_np(K.render_views(pos, col, op, sg, cfg, views, ctx=ctx))
    np.testing.assert_array_equal(got[0], got[2])
    single = to_np(K.render_views(pos, col, op, sg, cfg, (RenderViewPreset.Xy,), ctx=ctx))
    np.testing.assert_array_equal(got[1], single[0])
    _check_images(got, O.render_views(pos, col, op, sg, views, cfg), "render views Iso,Xy,Iso")
    empty = to_np(K.render_views(np.zeros((0, 4), np.float32), np.zeros((0, 3), np.float32),
                                 np.zeros(0, np.float32), np.zeros(0, np.float32), cfg, views, ctx=ctx))
    assert empty.shape == (3, 48, 48, 5) and not empty.any()
    far = pos.copy()
    far[:, :3] += 50.0  # every particle off every view
    assert not to_np(K.render_views(far, col, op, sg, cfg, ALL_VIEWS, ctx=ctx)).any()


def test_render_config_errors(ctx):
    """validate_render_loss_config (render_loss/attributes.rs:114-174) and this library's limits."""
    pos, col, op, sg = _particles(10, 1)
    cases = [(RenderLossConfig(sigma=0.0), "sigma must be finite and positive"),
             (RenderLossConfig(min_sigma=2.0, max_sigma=1.0), "max_sigma must be finite and >= min_sigma"),
             (RenderLossConfig(world_scale=float("nan")), "world_scale must be finite and positive"),
             (RenderLossConfig(image_size=0), "image_size must be non-zero"),
             (RenderLossConfig(target_samples=0), "target_samples must be non-zero"),
             (RenderLossConfig(depth_weight=-1.0), "depth_weight must be finite and non-negative"),
             (RenderLossConfig(max_sigma=400.0), "ceil(5*max_sigma) must be <= 1024")]
    for cfg, msg in cases:
        with pytest.raises(_abi.InvalidArgument, match=msg.replace("(", r"\(").replace(")", r"\)")
                           .replace("*", r"\*")):
            K.render_views(pos, col, op, sg, cfg, ALL_VIEWS, ctx=ctx)
    with pytest.raises(_abi.InvalidArgument, match="unknown render view 7"):
        K.render_views(pos, col, op, sg, RenderLossConfig(), (0, 7), ctx=ctx)
    with pytest.raises(_abi.InvalidArgument, match="1..=16 views"):
        K.render_views(pos, col, op, sg, RenderLossConfig(), [0] * 17, ctx=ctx)


@pytest.mark.parametrize("mode", list(GaussianDecodeMode))
def test_render_attributes_match_the_oracle(ctx, mode):
    rng = np.random.default_rng(int(mode) + 20)
    for S in (16, 9, 5, 4, 3):
        if mode == GaussianDecodeMode.GaussianSh0LearnedScale and S < 5:
            with pytest.raises(_abi.InvalidArgument, match="at least 5 state channels"):
                K.render_attributes(np.zeros((4, S), np.float32), S, RenderLossConfig(gaussian_decode_mode=mode),
                                    ctx=ctx)
            continue
        st = rng.normal(0, 3, (5000, S)).astype(np.float32)
        cfg = RenderLossConfig(gaussian_decode_mode=mode, sigma=2.0, min_sigma=0.5, max_sigma=6.0,
                               opacity_logit_bias=0.3)
        got = K.render_attributes(st, S, cfg, ctx=ctx)
        want = O.render_attributes(st, S, cfg)
        for g, w, name in zip(got, want, ("colors", "opacities", "sigmas", "derivatives")):
            assert rel_err(g, w) <= ATTR_TOL, (S, name)
        np.testing.assert_array_equal(to_np(got[0]), want[0])  # colours are exact
    with pytest.raises(_abi.InvalidArgument, match="at least 3 state channels"):
        K.render_attributes(np.zeros((4, 2), np.float32), 2, RenderLossConfig(), ctx=ctx)


@pytest.mark.parametrize("mode", [GaussianDecodeMode.GaussianSh0FixedScale,
                                  GaussianDecodeMode.GaussianSh0LearnedScale])
def test_state_render_views_after_a_c4_rollout(ctx, mode):
    """C4's 16,384 surface particles (S = 16: opacity channel 8, learned scale channel 11) after a
    16-step rollout, drawn in the four views from the device-resident state."""
    w = syn.workload("c4")
    steps = 16
    want_p, want_s = O.rollout(w["model"], w["weights"], w["positions"], w["states"], 1, w["n"], w["grid"],
                               steps, w["dt"], w["update_prob"], w["seed"], 0)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(w["model"], w["weights"]), w["positions"], w["states"], 1, w["n"],
                            w["grid"], w["dt"], w["update_prob"], w["seed"])
    ex.step_state_many(state, steps)
    gp, gs, _ = ex.read_state(state)
    gp, gs = to_np(gp), to_np(gs)
    assert rel_err(gp, want_p) <= 1e-3 and rel_err(gs, want_s) <= 1e-3
    cfg = RenderLossConfig(image_size=128, world_scale=0.8, gaussian_decode_mode=mode, opacity_logit_bias=0.5)
    got = ex.render_views(state, cfg)
    # the oracle draws the state the device holds
    col, op, sg, _ = O.render_attributes(gs, 16, cfg)
    want = O.render_views(gp, col, op, sg, ALL_VIEWS, cfg)
    _check_images(got, want, f"c4 state render ({mode.name})")
    state.close()


def test_state_render_needs_one_system(ctx):
    """validate_render_trace (render_loss/attributes.rs:89-112): batch_size must be 1."""
    w = syn.workload("c1", particles=256)
    ex = HipAutomataExecutor(ctx=ctx)
    pos = np.concatenate([w["positions"], w["positions"]])
    st = np.concatenate([w["states"], w["states"]])
    state = ex.create_state(NpaModel(w["model"], w["weights"]), pos, st, 2, 256, w["grid"], 1.0, 0.5, 1)
    with pytest.raises(_abi.InvalidArgument, match="expects batch_size=1, got 2"):
        ex.render_views(state, RenderLossConfig())
    state.close()
