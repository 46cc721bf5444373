"""The oriented Gaussian raster on the HIP path (npa_raster_gaussians_3d) against the CPU oracle.

The reference draws the planar Gaussian export through bevy_gaussian_splatting 8.0.1 (Cargo.toml:23;
crates/bevy_automata/src/viewer/cloud.rs:80-97), which is not vendored and whose pixels no
reference test pins (its headless test only asks for lit pixels,
crates/bevy_automata/tests/gaussian_gpu_link/headless.rs:4-58). Both sides restate the published 3D
Gaussian splatting forward pass; the oracle's restatement is pinned by closed forms in
tests/test_oracle.py. Bar: PSNR >= 90 dB against the oracle's image, at most 1 in 10^4 values off
by more than 1e-4 (the device's expf may differ from the host's by an ulp, which can move a pixel
across the 1/255 alpha floor or the 1e-4 transmittance cut).
"""
import math

import numpy as np
import pytest

from burn_automata_amd import _abi
from burn_automata_amd import kernels as K
from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import GaussianDecodeConfig, GaussianDecodeMode, RasterCamera, RasterColor
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel
from oracle import oracle as O
from tests.helpers import psnr, rel_err, to_np

pytestmark = pytest.mark.gpu

f32 = np.float32


def _check(got, want, what):
    g = to_np(got).astype(np.float64)
    w = np.asarray(want, np.float64)
    assert g.shape == w.shape, (g.shape, w.shape)
    d = np.abs(g - w)
    off = float((d > 1e-4).mean())
    p = psnr(g, w) if w.any() else (math.inf if not g.any() else 0.0)
    print(f"{what}: max diff {d.max():.3e}, rel err {rel_err(g, w):.2e}, values off by >1e-4 {off:.2e}, "
          f"psnr {p:.1f} dB, lit {float((w[..., 3] > 0).mean()):.2f}")
    assert p >= 90.0 and off <= 1e-4, what


def _cloud(n, degree, rng, spread=1.0, hidden=0.0):
    Kc = (degree + 1) ** 2
    pv = np.ones((n, 4), f32)
    pv[:, :3] = rng.uniform(-spread, spread, (n, 3))
    if hidden:
        pv[:, 3] = (rng.uniform(size=n) >= hidden).astype(f32)
    sh = rng.normal(0.0, 0.4, (n, Kc, 3)).astype(f32)
    rot = rng.normal(size=(n, 4)).astype(f32)
    so = np.empty((n, 4), f32)
    so[:, :3] = np.exp(rng.uniform(math.log(0.004), math.log(0.08), (n, 3)))
    so[:, 3] = rng.uniform(0.05, 1.0, n)
    return pv, sh, rot, so


CASES = {
    # name: (gaussians, width, height, sh degree, colour mode, eye, spread, hidden fraction)
    "one": (1, 64, 48, 0, RasterColor.Rgb, (0.0, 0.0, 3.0), 0.05, 0.0),
    "sh1_small": (500, 100, 75, 1, RasterColor.SphericalHarmonics, (0.5, 0.8, 3.0), 1.0, 0.1),
    "sh3_ragged": (5000, 257, 131, 3, RasterColor.SphericalHarmonics, (2.0, -1.0, 2.5), 1.0, 0.0),
    "rgb_1024": (40000, 1024, 1024, 0, RasterColor.Rgb, (0.0, 0.0, 3.5), 1.0, 0.05),
    "inside_the_cloud": (3000, 512, 384, 2, RasterColor.SphericalHarmonics, (0.1, 0.2, 0.6), 1.0, 0.0),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_raster_matches_the_oracle(ctx, name):
    """Random clouds: oriented anisotropic Gaussians, spherical harmonics of degree 0..3 or RGB,
    hidden ones, ragged edge tiles, and a camera inside the cloud (Gaussians behind it, beside it
    and covering most of the screen)."""
    n, W, H, deg, mode, eye, spread, hidden = CASES[name]
    rng = np.random.default_rng(len(name))
    pv, sh, rot, so = _cloud(n, deg, rng, spread, hidden)
    cam = RasterCamera.look_at(eye, width=W, height=H, sh_degree=deg, color_mode=mode)
    want = O.raster_gaussians_3d(pv, sh, rot, so, cam)
    got = K.raster_gaussians_3d(pv, sh, rot, so, cam, ctx=ctx)
    _check(got, want, f"raster {name} n={n} {W}x{H} deg={deg}")
    again = K.raster_gaussians_3d(pv, sh, rot, so, cam, ctx=ctx)
    np.testing.assert_array_equal(to_np(again), to_np(got))  # deterministic


def test_raster_equal_depth_ties(ctx):
    """Overlapping Gaussians on one plane facing the camera share a depth: the lower index is in
    front on both sides."""
    rng = np.random.default_rng(7)
    n = 400
    pv, sh, rot, so = _cloud(n, 0, rng)
    pv[:, 2] = 0.0
    pv[:, :2] = rng.uniform(-0.2, 0.2, (n, 2))
    so[:, 3] = 0.6
    cam = RasterCamera.look_at((0.0, 0.0, 2.0), width=128, height=128, color_mode=RasterColor.Rgb)
    want = O.raster_gaussians_3d(pv, sh, rot, so, cam)
    got = K.raster_gaussians_3d(pv, sh, rot, so, cam, ctx=ctx)
    _check(got, want, "equal depths")


def test_raster_empty_and_culled(ctx):
    cam = RasterCamera.look_at((0.0, 0.0, 3.0), width=40, height=24, far_plane=10.0)
    z = np.zeros((0, 4), f32)
    img = K.raster_gaussians_3d(z, np.zeros(0, f32), z, z, cam, ctx=ctx)
    assert img.shape == (24, 40, 4) and not to_np(img).any()
    pv = np.array([[0, 0, 0, 0.0], [0, 0, 4, 1.0], [0, 0, -8, 1.0]], f32)  # hidden, behind, beyond far
    so = np.full((3, 4), 0.5, f32)
    rot = np.tile(np.array([1, 0, 0, 0], f32), (3, 1))
    img = K.raster_gaussians_3d(pv, np.ones((3, 3), f32), rot, so, cam, ctx=ctx)
    assert not to_np(img).any()


@pytest.mark.parametrize("mode", [GaussianDecodeMode.GaussianSh0FixedScale, GaussianDecodeMode.GaussianSh0Oriented,
                                  None])
def test_state_raster_after_a_c4_rollout(ctx, mode):
    """C4's 16,384 surface particles after 8 steps: the frame of the device-resident state (decode or
    viewer export, then raster, in one call) equals the oracle's raster of the same Gaussians. A decode
    config draws the decoded colours as RGB; no config draws the viewer's export (48 SH coefficients,
    evaluated at degree 3)."""
    w = syn.workload("c4")
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(w["model"], w["weights"]), w["positions"], w["states"], 1, w["n"],
                            w["grid"], w["dt"], w["update_prob"], w["seed"])
    ex.step_state_many(state, 8)
    if mode is None:
        dcfg = None
        gp, gs, _ = ex.read_state(state)
        dec = O.write_gaussians(to_np(gp), to_np(gs), w["n"], w["model"], w["grid"])
        dec["spherical_harmonic"] = dec["spherical_harmonic"].reshape(-1, 16, 3)
        color, deg = RasterColor.SphericalHarmonics, 3
    else:
        dcfg = GaussianDecodeConfig(mode=mode)
        dec = {k: to_np(v) for k, v in ex.decode_gaussians_3d(state, dcfg).items()}
        color, deg = RasterColor.Rgb, 0
    p = dec["position_visibility"][:, :3]
    centre = p.mean(axis=0)
    ext = float(np.abs(p - centre).max())
    eye = tuple(centre + np.array([0.6, 0.9, 2.4]) * ext)
    cam = RasterCamera.look_at(eye, tuple(centre), width=320, height=240)  # default colour mode
    got = ex.raster_gaussians_3d(state, dcfg, cam)
    want = O.raster_gaussians_3d(dec["position_visibility"], dec["spherical_harmonic"], dec["rotation"],
                                 dec["scale_opacity"], cam.replace(color_mode=color, sh_degree=deg))
    _check(got, want, f"c4 state raster ({mode.name if mode else 'viewer export'})")
    assert float((want[..., 3] > 0.01).mean()) > 0.05  # the surface is in view
    state.close()


@pytest.mark.parametrize("sh_degree,S", [(1, 20), (1, 32)])
def test_state_raster_oriented_decode_above_degree_zero(ctx, sh_degree, S):
    """An oriented decode of SH degree d stores (d + 1)^2 coefficient triples per Gaussian, the colour
    in the first: the state raster must read every Gaussian's colour at that stride (S >= 3 (d + 1)^2
    + 8; the device path takes up to 32 state channels, so degree 1 is the largest such decode of a
    state), after a few steps of the two-kernel path."""
    from burn_automata_amd.config import HashGridConfig, NpaConfig

    m = NpaConfig.growing_3dgs().replace(state_dims=S)
    g = HashGridConfig.growing_3dgs()
    n = 1500
    pos = syn.uniform_ball(n, 71, 0.5)
    st = syn.normal_states(n, S, 71, std=0.5)
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, syn.seeded_weights(m, 71)), pos, st, 1, n, g, 1.0, 0.5, 42)
    ex.step_state_many(state, 3)
    dcfg = GaussianDecodeConfig(mode=GaussianDecodeMode.GaussianSh0Oriented, sh_degree=sh_degree)
    dec = {k: to_np(v) for k, v in ex.decode_gaussians_3d(state, dcfg).items()}
    Kc = (sh_degree + 1) ** 2
    assert dec["spherical_harmonic"].reshape(n, -1).shape[1] == Kc * 3
    colours = np.ascontiguousarray(dec["spherical_harmonic"].reshape(n, Kc, 3)[:, :1, :])
    cam = RasterCamera.look_at((0.4, 0.7, 1.8), width=160, height=120)
    got = ex.raster_gaussians_3d(state, dcfg, cam)
    want = O.raster_gaussians_3d(dec["position_visibility"], colours, dec["rotation"], dec["scale_opacity"],
                                 cam.replace(color_mode=RasterColor.Rgb, sh_degree=0))
    _check(got, want, f"state raster, oriented decode at SH degree {sh_degree}")
    assert float((want[..., 3] > 0.01).mean()) > 0.05
    # the coefficients past the first differ from the colour, so a wrong stride would change pixels
    assert not np.array_equal(dec["spherical_harmonic"].reshape(n, Kc, 3)[:, 1], colours[:, 0])
    state.close()


def test_state_raster_default_camera_keeps_the_decoded_colour(ctx):
    """One opaque particle in front of a default camera (colour mode SH): the state raster draws its
    decoded colour clamp(tail + 0.5), not 0.5 + SH_C0 * colour, both from the decode (RGB) and from
    the viewer export (whose DC coefficient (c - 0.5) / SH_C0 evaluates back to c)."""
    from burn_automata_amd.config import HashGridConfig, NpaConfig

    m = NpaConfig.growing_3dgs().replace(state_dims=12, hidden_dims=8)
    g = HashGridConfig.growing_3dgs()
    rgb = np.array([0.35, -0.2, 0.1], f32)  # tail: colours 0.85, 0.3, 0.6
    st = np.zeros((1, m.state_dims), f32)
    st[0, -3:] = rgb
    st[0, 8] = 8.0  # opacity logit: sigmoid(8) clamps to 0.95
    pos = np.zeros((1, 4), f32)
    weights = {k: np.zeros(v, f32) for k, v in (("w1", m.hidden_dims * m.perception_dims()),
                                                ("b1", m.hidden_dims),
                                                ("w2", m.update_dims() * m.hidden_dims),
                                                ("b2", m.update_dims()))}
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, weights), pos, st, 1, 1, g, 1.0, 1.0, 0)
    cam = RasterCamera.look_at((0.0, 0.0, 1.0), width=33, height=33)
    assert cam.color_mode == RasterColor.SphericalHarmonics
    want = np.clip(rgb + 0.5, 0, 1)
    for dcfg in (GaussianDecodeConfig(mode=GaussianDecodeMode.GaussianSh0FixedScale, sigma=0.2, opacity_scale=0.95,
                                      max_opacity=0.95), None):
        img = to_np(ex.raster_gaussians_3d(state, dcfg, cam))
        centre = img[16, 16]
        assert centre[3] > 0.5
        np.testing.assert_allclose(centre[:3] / centre[3], want, rtol=1e-5, atol=1e-6)
    state.close()


def test_raster_errors(ctx):
    pv, sh, rot, so = _cloud(4, 0, np.random.default_rng(1))
    cam = RasterCamera.look_at((0.0, 0.0, 3.0), width=32, height=32)
    for bad, msg in ((cam.replace(width=0), "non-zero"), (cam.replace(sh_degree=4), "sh_degree"),
                     (cam.replace(near_plane=0.0), "near_plane"), (cam.replace(far_plane=0.05), "far_plane"),
                     (cam.replace(width=16384, height=16384), "65536"), (cam.replace(fx=-1.0), "focal"),
                     (cam.replace(width=20000), "16384")):
        shb = np.zeros(4 * (bad.sh_degree + 1) ** 2 * 3, f32)  # sized for the camera's degree
        with pytest.raises(_abi.InvalidArgument, match=msg):
            K.raster_gaussians_3d(pv, shb, rot, so, bad, ctx=ctx)
    with pytest.raises(AssertionError, match="differ in length"):
        K.raster_gaussians_3d(pv, sh[:3], rot, so, cam, ctx=ctx)
