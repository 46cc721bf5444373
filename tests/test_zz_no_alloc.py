"""npa_step_noalloc: npa_step with its workspace in a fixed device array (no allocation).

Called through the C ABI and compared with npa_step on the same inputs, bit for bit, over calls in
a row on one GPU: the array keeps the previous call's contents, so the second call is smaller than
the first (a leftover of the larger system must not leak into it) and the third is the C2 system
the header says fits. Systems whose workspace exceeds the array, and host-I/O mode, are refused
before any work is queued.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from burn_automata_amd import _abi
from burn_automata_amd import synthetic as syn
from burn_automata_amd._lib import lib
from burn_automata_amd.model import NpaWeights
from burn_automata_amd.runtime import Context, device_f32, ptr
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _run(ctx, fn, w, mask):
    m, g, b, n = w["model"], w["grid"], w["batch"], w["n"]
    total = b * n
    pos = device_f32(w["positions"]).reshape(-1, 4)
    st = device_f32(w["states"]).reshape(-1)
    msk = None if mask is None else device_f32(mask)
    weights = NpaWeights.from_arrays(w["weights"])
    wc = weights.to_c()
    out_p = torch.full_like(pos, float("nan"))
    out_s = torch.full_like(st, float("nan"))
    dens = torch.full((total,), float("nan"), dtype=torch.float32, device=pos.device)
    code = fn(ctx.handle, ptr(pos), ptr(st), b, n, C.byref(g.to_c()), C.byref(m.to_c()), C.byref(wc), 1.0,
              ptr(msk), ptr(out_p), ptr(out_s), ptr(dens))
    ctx.check(code)
    ctx.synchronize()
    return out_p.cpu().numpy(), out_s.cpu().numpy(), dens.cpu().numpy()


def _case(name, particles, masked):
    w = syn.workload(name, particles=particles)
    mask = O.update_mask(w["batch"], w["n"], 0.5, 3, w["seed"]) if masked else None
    return w, mask


def test_noalloc_step_equals_npa_step_on_calls_in_a_row(ctx):
    L = lib()
    # larger, then smaller (the array still holds the first call's workspace), then the C2 system;
    # then C4's sparse 3D grid twice (the binned build, whose bin counters the call clears itself)
    for name, particles, masked in (("c1", 4096, True), ("c1", 1024, False), ("c5", 256, True),
                                    ("c2", None, True), ("c4", None, True), ("c4", 6000, False)):
        w, mask = _case(name, particles, masked)
        print(f"noalloc vs npa_step: {name} batch={w['batch']} n={w['n']} masked={masked}", flush=True)
        want = _run(ctx, L.npa_step, w, mask)
        got = _run(ctx, L.npa_step_noalloc, w, mask)
        for k, (a, b) in enumerate(zip(got, want)):
            assert np.isfinite(b).all(), (name, k)
            np.testing.assert_array_equal(a, b, err_msg=f"{name} output {k}")


def test_noalloc_refuses_oversized_systems_and_host_io(ctx):
    L = lib()
    # C5's 64 systems of 4,096 particles on per-system 64x64 grids need more than 100 MiB of
    # workspace (about 450 bytes per particle), well over the 64 MiB array
    w = syn.workload("c5")
    m, g, b, n = w["model"], w["grid"], w["batch"], w["n"]
    wc = NpaWeights.from_arrays(w["weights"]).to_c()
    pos = device_f32(w["positions"]).reshape(-1, 4)
    st = device_f32(w["states"]).reshape(-1)
    out_p, out_s = torch.empty_like(pos), torch.empty_like(st)
    code = L.npa_step_noalloc(ctx.handle, ptr(pos), ptr(st), b, n, C.byref(g.to_c()), C.byref(m.to_c()),
                              C.byref(wc), 1.0, None, ptr(out_p), ptr(out_s), None)
    msg = L.npa_last_error(ctx.handle).decode()
    assert code == _abi.NPA_ERR_INVALID_ARGUMENT and "bytes of workspace" in msg, (code, msg)
    # host-I/O mode stages through allocations: refused
    hctx = Context(0, host_io=True)
    hp = np.ascontiguousarray(w["positions"][:n], np.float32)
    hs = np.ascontiguousarray(w["states"][:n], np.float32)
    ho_p, ho_s = np.zeros_like(hp), np.zeros_like(hs)
    host_w = [np.ascontiguousarray(w["weights"][k], np.float32).ravel() for k in ("w1", "b1", "w2", "b2")]
    hwc = _abi.NpaWeightsC(*(a.ctypes.data_as(C.c_void_p) for a in host_w))
    code = L.npa_step_noalloc(hctx.handle, hp.ctypes.data_as(C.c_void_p), hs.ctypes.data_as(C.c_void_p), 1, n,
                              C.byref(g.to_c()), C.byref(m.to_c()), C.byref(hwc), 1.0, None,
                              ho_p.ctypes.data_as(C.c_void_p), ho_s.ctypes.data_as(C.c_void_p), None)
    assert code == _abi.NPA_ERR_INVALID_ARGUMENT
    hctx.close()
    ctx.synchronize()


@pytest.mark.parametrize("name,particles", [("c1", 4096), ("c4", None)])
def test_noalloc_step_replays_in_a_hip_graph(ctx, name, particles):
    """npa_step_noalloc queues kernels only (no allocation, no memset node, no host wait), so a
    caller can capture it: captured once through torch.cuda.graph on the capture stream, every
    replay - with eager work and synchronisation in between - equals the eager call bit for bit."""
    L = lib()
    w, mask = _case(name, particles, True)
    m, g, b, n = w["model"], w["grid"], w["batch"], w["n"]
    total = b * n
    pos = device_f32(w["positions"]).reshape(-1, 4)
    st = device_f32(w["states"]).reshape(-1)
    msk = device_f32(mask)
    weights = NpaWeights.from_arrays(w["weights"])  # holds the weight tensors the graph reads
    wc = weights.to_c()
    gc, mc = g.to_c(), m.to_c()
    out_p, out_s = torch.empty_like(pos), torch.empty_like(st)
    dens = torch.empty((total,), dtype=torch.float32, device=pos.device)

    def call():
        return L.npa_step_noalloc(ctx.handle, ptr(pos), ptr(st), b, n, C.byref(gc), C.byref(mc), C.byref(wc), 1.0,
                                  ptr(msk), ptr(out_p), ptr(out_s), ptr(dens))

    print(f"graph capture of npa_step_noalloc: {name} n={total}", flush=True)
    ctx.check(call())  # eager (also sets the kernels' LDS limits, outside the capture)
    ctx.synchronize()
    want = [t.cpu().numpy().copy() for t in (out_p, out_s, dens)]
    graph = torch.cuda.CUDAGraph()
    home = torch.cuda.current_stream().cuda_stream
    try:
        with torch.cuda.graph(graph):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            code = call()
    finally:
        ctx.set_stream(home)
    ctx.check(code)
    for k in range(3):
        for t in (out_p, out_s, dens):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for t, ref in zip((out_p, out_s, dens), want):
            np.testing.assert_array_equal(t.cpu().numpy(), ref, err_msg=f"{name} replay {k}")
