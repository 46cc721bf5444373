"""Host-I/O mode (npa_context_set_host_io): the C-ABI called with host pointers.

A context in host-I/O mode stages host inputs to the device and copies the outputs back before the
call returns; the results must equal the same call's on device pointers bit for bit (the same
kernels run on the same values). Covered here through the raw C-ABI with numpy arrays: the
Gaussian decode, the 2D splat, the projected render, the oriented raster and the rollout step.
"""
import ctypes as C

import numpy as np
import pytest

from burn_automata_amd import kernels as K
from burn_automata_amd._lib import lib
from burn_automata_amd.config import (ALL_VIEWS, GaussianDecodeConfig, GaussianDecodeMode, RasterCamera,
                                      RasterColor, RenderLossConfig, Splat2dConfig)
from burn_automata_amd.runtime import Context
from tests.helpers import to_np

pytestmark = pytest.mark.gpu

f32 = np.float32


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.fixture(scope="module")
def host_ctx():
    c = Context(host_io=True)
    yield c
    c.close()


def _inputs(n=2000, S=16, seed=3):
    rng = np.random.default_rng(seed)
    pos = np.zeros((n, 4), f32)
    pos[:, :3] = rng.uniform(-0.8, 0.8, (n, 3))
    st = rng.normal(0, 0.4, (n, S)).astype(f32)
    return pos, st


def test_decode_and_raster_on_host_pointers(ctx, host_ctx):
    pos, st = _inputs()
    n, S = pos.shape[0], st.shape[1]
    cfg = GaussianDecodeConfig(mode=GaussianDecodeMode.GaussianSh0Oriented)
    pv, sh = np.zeros((n, 4), f32), np.zeros((n, 1, 3), f32)
    rot, so = np.zeros((n, 4), f32), np.zeros((n, 4), f32)
    host_ctx.check(lib().npa_decode_gaussians_3d(host_ctx.handle, _p(pos), _p(st), n, S, C.byref(cfg.to_c()),
                                                 _p(pv), _p(sh), _p(rot), _p(so)))
    want = K.decode_gaussians_3d(pos, st, S, cfg, ctx=ctx)
    for k, got in (("position_visibility", pv), ("spherical_harmonic", sh), ("rotation", rot),
                   ("scale_opacity", so)):
        np.testing.assert_array_equal(got, to_np(want[k]).reshape(got.shape), err_msg=k)
    cam = RasterCamera.look_at((0.5, 0.7, 2.5), width=200, height=150, color_mode=RasterColor.SphericalHarmonics)
    img = np.zeros((150, 200, 4), f32)
    host_ctx.check(lib().npa_raster_gaussians_3d(host_ctx.handle, _p(pv), _p(sh), _p(rot), _p(so), n,
                                                 C.byref(cam.to_c()), _p(img)))
    dev = K.raster_gaussians_3d(pv, sh, rot, so, cam, ctx=ctx)
    np.testing.assert_array_equal(img, to_np(dev))
    assert img[..., 3].max() > 0.1


def test_splat_and_render_on_host_pointers(ctx, host_ctx):
    pos, st = _inputs(seed=5)
    n = pos.shape[0]
    col = np.clip(st[:, -3:] + 0.5, 0, 1).astype(f32)
    scfg = Splat2dConfig(image_size=96)
    img = np.zeros((96 * 96, 4), f32)
    host_ctx.check(lib().npa_splat_2d(host_ctx.handle, _p(pos), _p(col), n, C.byref(scfg.to_c()), _p(img)))
    np.testing.assert_array_equal(img.reshape(-1), to_np(K.splat_particles_2d(pos, col, scfg, ctx=ctx)).reshape(-1))
    rcfg = RenderLossConfig(image_size=48)
    op = np.full(n, 0.6, f32)
    sg = np.full(n, 2.0, f32)
    views = np.array([int(v) for v in ALL_VIEWS], np.uint32)
    imgs = np.zeros((len(views), 48, 48, 5), f32)
    host_ctx.check(lib().npa_render_views(host_ctx.handle, _p(pos), _p(col), _p(op), _p(sg), n, _p(views),
                                          len(views), C.byref(rcfg.to_c()), _p(imgs)))
    np.testing.assert_array_equal(imgs, to_np(K.render_views(pos, col, op, sg, rcfg, ctx=ctx)))


def test_step_on_host_pointers(ctx, host_ctx):
    """npa_step (NpaModel::step_cpu, model.rs:768-858) with host positions, states, mask, weights and
    outputs: equal to the device-pointer step bit for bit."""
    from burn_automata_amd import _abi
    from burn_automata_amd import synthetic as syn
    from burn_automata_amd.model import NpaModel

    w = syn.workload("c1", particles=2048)
    model = NpaModel(w["model"], w["weights"])
    n, S = w["n"], w["model"].state_dims
    pos = np.ascontiguousarray(w["positions"], f32)
    st = np.ascontiguousarray(w["states"], f32).reshape(-1)
    mask = (np.random.default_rng(9).uniform(size=n) < 0.5).astype(f32)
    dev = model.step(pos, st, 1, n, w["grid"], w["dt"], mask, ctx=ctx)
    W = model.weights
    w1, b1, w2, b2 = (np.ascontiguousarray(to_np(a), f32) for a in (W.w1, W.b1, W.w2, W.b2))
    wc = _abi.NpaWeightsC(_p(w1), _p(b1), _p(w2), _p(b2))
    op, os_, dens = np.zeros((n, 4), f32), np.zeros(n * S, f32), np.zeros(n, f32)
    host_ctx.check(lib().npa_step(host_ctx.handle, _p(pos), _p(st), 1, n, C.byref(w["grid"].to_c()),
                                  C.byref(model.config.to_c()), C.byref(wc), float(w["dt"]), _p(mask), _p(op),
                                  _p(os_), _p(dens)))
    np.testing.assert_array_equal(op, to_np(dev.next_positions))
    np.testing.assert_array_equal(os_.reshape(n, S), to_np(dev.next_states))
    np.testing.assert_array_equal(dens, to_np(dev.density))
    assert not np.array_equal(os_, st)  # the step changed the states
