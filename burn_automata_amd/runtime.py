"""Context handle over the C ABI, plus tensor plumbing (torch for device memory only)."""
from __future__ import annotations

import ctypes as C

from . import _abi
from ._lib import lib


class Context:
    """An ``npa_context`` bound to one device and one HIP stream.

    By default the context runs on torch's current stream of ``device`` so the
    library's launches order with torch work on that stream.
    """

    def __init__(self, device: int = 0, stream=None, host_io: bool = False):
        import torch

        L = lib()
        if stream is None:
            stream = torch.cuda.current_stream(device).cuda_stream
        handle = C.c_void_p()
        code = L.npa_context_create(int(device), C.c_void_p(stream), C.byref(handle))
        if code:
            raise _abi.error_for(code, f"npa_context_create(device={device}) failed")
        self.handle = handle
        self.device = device
        self._host_io = False
        if host_io:
            self.host_io = True

    @property
    def host_io(self) -> bool:
        return self._host_io

    @host_io.setter
    def host_io(self, value: bool):
        self.check(lib().npa_context_set_host_io(self.handle, int(bool(value))))
        self._host_io = bool(value)

    def set_mlp_engine(self, engine: int):
        """npa_step's update-MLP engine: MLP_VALU (bit-exact, default) or MLP_MFMA."""
        self.check(lib().npa_context_set_mlp_engine(self.handle, int(engine)))

    def set_stream(self, stream):
        self.check(lib().npa_context_set_stream(self.handle, C.c_void_p(stream)))

    def check(self, code: int):
        if code:
            msg = lib().npa_last_error(self.handle)
            raise _abi.error_for(code, msg.decode() if msg else "")

    def synchronize(self):
        self.check(lib().npa_context_synchronize(self.handle))

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle.value:
            lib().npa_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_DEFAULT: dict = {}


def default_context(device: int = 0) -> Context:
    ctx = _DEFAULT.get(device)
    if ctx is None:
        ctx = Context(device)
        _DEFAULT[device] = ctx
    return ctx


def version() -> str:
    return lib().npa_version().decode()


def device_f32(x, shape=None, device: int = 0):
    """A contiguous float32 CUDA tensor view/copy of ``x`` (torch tensor or array-like)."""
    import numpy as np
    import torch

    if isinstance(x, torch.Tensor):
        t = x
        if t.device.type != "cuda":
            t = t.to(f"cuda:{device}")
        if t.dtype != torch.float32:
            t = t.float()
    else:
        t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(f"cuda:{device}")
    t = t.contiguous()
    if shape is not None:
        t = t.reshape(shape)
    return t


def ptr(t) -> C.c_void_p:
    return C.c_void_p(0 if t is None else t.data_ptr())
