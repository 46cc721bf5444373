"""Error paths of the C ABI on the device: null arrays and coordinate overflow.

A null array that a call reads or writes is refused with NPA_ERR_INVALID_ARGUMENT before any
device work is queued (every other array of these calls is a valid device buffer of the right
size). NPA_ERR_COORD_OVERFLOW: a Particle-mode cell coordinate beyond +-2^30 is returned by the
call itself in host-I/O mode and by the next synchronising call in device-pointer mode, and is
cleared once reported.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from burn_automata_amd import _abi
from burn_automata_amd import kernels as K
from burn_automata_amd import synthetic as syn
from burn_automata_amd._lib import lib
from burn_automata_amd.config import GaussianDecodeConfig
from burn_automata_amd.executor import HipAutomataExecutor
from burn_automata_amd.model import NpaModel, NpaWeights
from burn_automata_amd.runtime import Context, ptr

pytestmark = pytest.mark.gpu

NULL = C.c_void_p(0)


def _dev(shape):
    return torch.zeros(shape, dtype=torch.float32, device="cuda:0")


def _case(n=256):
    w = syn.workload("c1", particles=n)
    return w["model"], w["grid"], w["positions"], w["states"], w["weights"], n


def _status(ctx, code):
    return code, lib().npa_last_error(ctx.handle).decode()


def test_null_arrays_are_refused_before_any_launch(ctx):
    m, g, pos, st, w, n = _case()
    S, F, H, O = m.state_dims, m.perception_dims(), m.hidden_dims, m.update_dims()
    L = lib()
    dpos, dst = _dev((n, 4)), _dev((n, S))
    dpos.copy_(torch.from_numpy(pos))
    dst.copy_(torch.from_numpy(st.reshape(n, S)))
    out_p, out_s, dens = _dev((n, 4)), _dev((n, S)), _dev(n)
    weights = NpaWeights.from_arrays(w, 0)
    wc = weights.to_c()
    gc, mc = g.to_c(), m.to_c()
    arrays = [dpos, dst, out_p, out_s]
    for k in range(len(arrays)):
        args = [ptr(a) for a in arrays]
        args[k] = NULL
        code, msg = _status(ctx, L.npa_step(ctx.handle, args[0], args[1], 1, n, C.byref(gc), C.byref(mc),
                                            C.byref(wc), 1.0, NULL, args[2], args[3], ptr(dens)))
        assert code == _abi.NPA_ERR_INVALID_ARGUMENT and "null" in msg, (k, code, msg)
    for field in ("w1", "b1", "w2", "b2"):
        bad = weights.to_c()
        setattr(bad, field, None)
        code, msg = _status(ctx, L.npa_step(ctx.handle, ptr(dpos), ptr(dst), 1, n, C.byref(gc), C.byref(mc),
                                            C.byref(bad), 1.0, NULL, ptr(out_p), ptr(out_s), NULL))
        assert code == _abi.NPA_ERR_INVALID_ARGUMENT and "null" in msg, (field, code, msg)
    # euler_step: positions, states, dx, ds and both outputs
    dx, ds = _dev((n, 4)), _dev((n, S))
    arrays = [dpos, dst, dx, ds, out_p, out_s]
    for k in range(len(arrays)):
        args = [ptr(a) for a in arrays]
        args[k] = NULL
        code = L.npa_euler_step(ctx.handle, args[0], args[1], args[2], args[3], 1, n, S, C.byref(gc),
                                1.0, NULL, args[4], args[5])
        assert code == _abi.NPA_ERR_INVALID_ARGUMENT, (k, code)
    # mlp_forward: features and both outputs
    feats = _dev((n, F))
    arrays = [feats, dx, ds]
    for k in range(len(arrays)):
        args = [ptr(a) for a in arrays]
        args[k] = NULL
        code = L.npa_mlp_forward(ctx.handle, args[0], n, C.byref(mc), C.byref(wc), 0.05, args[1], args[2])
        assert code == _abi.NPA_ERR_INVALID_ARGUMENT, (k, code)
    # decode_gaussians_3d: positions, states and the four outputs
    dcfg = GaussianDecodeConfig().to_c()
    outs = [_dev((n, 4)), _dev((n, 1, 3)), _dev((n, 4)), _dev((n, 4))]
    arrays = [dpos, dst] + outs
    for k in range(len(arrays)):
        args = [ptr(a) for a in arrays]
        args[k] = NULL
        code = L.npa_decode_gaussians_3d(ctx.handle, args[0], args[1], n, S, C.byref(dcfg), *args[2:])
        assert code == _abi.NPA_ERR_INVALID_ARGUMENT, (k, code)
    # neighbor_lists: positions
    offsets = torch.zeros(n + 1, dtype=torch.int32, device="cuda:0")
    req = C.c_size_t()
    code = L.npa_neighbor_lists(ctx.handle, NULL, 1, n, C.byref(gc), ptr(offsets), NULL, 0, C.byref(req))
    assert code == _abi.NPA_ERR_INVALID_ARGUMENT
    # update_mask: the mask
    assert L.npa_update_mask(ctx.handle, 1, n, 0.5, 0, 42, NULL) == _abi.NPA_ERR_INVALID_ARGUMENT
    # a state's decode outputs
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(NpaModel(m, w), pos, st, 1, n, g, 1.0, 0.5, 42)
    for k in range(4):
        args = [ptr(a) for a in outs]
        args[k] = NULL
        code = L.npa_state_decode_gaussians_3d(state.handle, C.byref(dcfg), *args)
        assert code == _abi.NPA_ERR_INVALID_ARGUMENT, (k, code)
    # nothing was queued: the state steps and reads back normally
    ex.step_state(state)
    ctx.synchronize()
    state.close()


def _far_positions(pos, g):
    """Particles past the +-2^30-cell range a Particle grid stores exactly (x = 1e8 at eps 0.05 is
    cell 2e9)."""
    far = np.array(pos, np.float32, copy=True)
    far[::17, 0] = np.float32(1e8)
    far[5::17, 1] = np.float32(-1e8)
    assert np.max(np.abs(far[:, :2])) / g.eps > 2 ** 30
    return far


def test_coord_overflow_host_io_reported_then_cleared():
    m, g, pos, st, w, n = _case()
    hctx = Context(0, host_io=True)
    far = _far_positions(pos, g)
    bo = np.zeros(g.cell_count() + 1, np.uint32)
    perm = np.zeros(n, np.uint32)
    inv = np.zeros(n, np.uint32)

    def hashgrid(positions):
        p = np.ascontiguousarray(positions, np.float32)
        return lib().npa_build_hashgrid(hctx.handle, p.ctypes.data_as(C.c_void_p), 1, n, C.byref(g.to_c()),
                                        bo.ctypes.data_as(C.c_void_p), bo.size, perm.ctypes.data_as(C.c_void_p),
                                        inv.ctypes.data_as(C.c_void_p), n)

    assert hashgrid(far) == _abi.NPA_ERR_COORD_OVERFLOW
    assert hashgrid(pos) == 0  # clean data: no stale report
    out_p = np.zeros((n, 4), np.float32)
    out_s = np.zeros((n, m.state_dims), np.float32)
    host_w = [np.ascontiguousarray(w[k], np.float32).ravel() for k in ("w1", "b1", "w2", "b2")]
    wc = _abi.NpaWeightsC(*(a.ctypes.data_as(C.c_void_p) for a in host_w))
    for positions, want in ((far, _abi.NPA_ERR_COORD_OVERFLOW), (pos, 0)):
        p = np.ascontiguousarray(positions, np.float32)
        s = np.ascontiguousarray(st, np.float32)
        code = lib().npa_step(hctx.handle, p.ctypes.data_as(C.c_void_p), s.ctypes.data_as(C.c_void_p), 1, n,
                              C.byref(g.to_c()), C.byref(m.to_c()), C.byref(wc), 1.0, NULL,
                              out_p.ctypes.data_as(C.c_void_p), out_s.ctypes.data_as(C.c_void_p), NULL)
        assert code == want
    hctx.close()


def test_coord_overflow_device_mode_reported_at_synchronize(ctx):
    m, g, pos, st, w, n = _case()
    model = NpaModel(m, w)
    far = _far_positions(pos, g)
    model.step(far, st, 1, n, g, 1.0, ctx=ctx)  # queued: returns without waiting
    with pytest.raises(_abi.CoordOverflow):
        ctx.synchronize()
    ctx.synchronize()  # reported once, then cleared
    with pytest.raises(_abi.CoordOverflow):
        K.neighbor_lists(far, 1, n, g, ctx=ctx)  # synchronises: reports its own build
    ex = HipAutomataExecutor(ctx=ctx)
    state = ex.create_state(model, far, st, 1, n, g, 1.0, 0.5, 42)
    ex.step_state(state)
    with pytest.raises(_abi.CoordOverflow):
        ex.read_state(state)
    ex.read_state(state)  # cleared
    state.close()
