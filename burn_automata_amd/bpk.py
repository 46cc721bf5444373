"""`.bpk` model files (crates/burn_automata/src/import.rs:16-36, 378-506) through libnpa_hip.so.

``load_manifest`` / ``load_manifest_bytes`` / ``decode_bpk_manifest`` read a container or its bare
JSON payload with the reference's checks (header, magic, version, length, SHA-256, JSON,
validate_manifest) and return a :class:`BpkModelManifest` whose ``into_model()`` is an
:class:`NpaModel` ready for the HIP step and executor. ``encode_bpk_manifest`` wraps a serialized
payload in a container. All of it is host code in the library; no device is touched.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _abi
from ._lib import lib
from .config import Boundary, EquivarianceMode, HashGridConfig, HashGridMode, NpaConfig

BPK_MAGIC = b"BAUTBPK1"
BPK_HEADER_LEN = 8 + 4 + 8 + 32


@dataclass
class BpkModelManifest:
    """BpkModelManifest (import.rs:20-31); weights as float32 numpy arrays."""

    format_version: int
    model_kind: str
    source: str | None
    config: NpaConfig
    hashgrid: HashGridConfig
    weights: dict
    initialization: tuple | None  # (positions [n, 4], states [n * S]) or None
    auxiliary_input_dims: int = 0
    decoder_dims: int | None = None
    output_dims: int | None = None

    def into_model(self, device: int = 0):
        """BpkModelManifest::into_model (import.rs:94-99)."""
        from .model import NpaModel

        return NpaModel(self.config, self.weights, device)


def _load(handle_fn) -> BpkModelManifest:
    L = lib()
    h = C.c_void_p()
    err = C.create_string_buffer(512)
    code = handle_fn(C.byref(h), err)
    if code:
        raise _abi.error_for(code, err.value.decode(errors="replace"))
    try:
        info = _abi.NpaManifestInfo()
        _check(L.npa_manifest_info(h, C.byref(info)))
        m, g, w = _abi.NpaModelCfg(), _abi.NpaGridCfg(), _abi.NpaWeightsC()
        code = L.npa_manifest_model(h, C.byref(m), C.byref(g), C.byref(w))
        if code == _abi.NPA_ERR_INVALID_MODEL:  # auxiliary inputs: kept as data, not runnable
            L.npa_manifest_model(h, None, C.byref(g), None)
            raise _abi.InvalidModel("manifest has auxiliary input dims "
                                    f"{info.auxiliary_input_dims}; the rollout path takes none")
        _check(code)
        config = NpaConfig(spatial_dims=m.spatial_dims, state_dims=m.state_dims,
                           hidden_dims=m.hidden_dims, eps0=m.eps0, alpha=m.alpha,
                           density_grad=bool(m.density_grad), state_grad=bool(m.state_grad),
                           log_norm_grad=bool(m.log_norm_grad),
                           log_norm_density_grad=bool(m.log_norm_density_grad),
                           equivariance=EquivarianceMode(m.equivariance),
                           position_features=bool(m.position_features))
        grid = HashGridConfig(int(g.dim), Boundary(g.boundary), HashGridMode(g.mode),
                              tuple(int(v) for v in g.grid_size), float(g.eps),
                              int(g.max_particles_per_block))
        F, H, O = config.perception_dims(), config.hidden_dims, config.update_dims()
        weights = {k: _copy(getattr(w, k), n) for k, n in
                   (("w1", H * F), ("b1", H), ("w2", O * H), ("b2", O))}
        init = None
        if info.initialization_particles:
            p, s, n = C.c_void_p(), C.c_void_p(), C.c_uint32()
            _check(L.npa_manifest_initialization(h, C.byref(p), C.byref(s), C.byref(n)))
            init = (_copy(p.value, 4 * n.value).reshape(-1, 4),
                    _copy(s.value, n.value * config.state_dims))
        return BpkModelManifest(
            format_version=int(info.format_version), model_kind=info.model_kind.decode(),
            source=info.source.decode() if info.source is not None else None, config=config,
            hashgrid=grid, weights=weights, initialization=init,
            auxiliary_input_dims=int(info.auxiliary_input_dims),
            decoder_dims=None if info.decoder_dims < 0 else int(info.decoder_dims),
            output_dims=None if info.output_dims < 0 else int(info.output_dims))
    finally:
        L.npa_manifest_destroy(h)


def _copy(addr, n) -> np.ndarray:
    if n == 0:
        return np.zeros(0, np.float32)
    buf = (C.c_float * n).from_address(addr if isinstance(addr, int) else addr.value)
    return np.frombuffer(buf, dtype=np.float32, count=n).copy()


def _check(code):
    if code:
        raise _abi.error_for(code)


def load_manifest_bytes(data: bytes) -> BpkModelManifest:
    """load_manifest_bytes (import.rs:383-390): a .bpk container or the bare JSON manifest."""
    data = bytes(data)
    return _load(lambda h, err: lib().npa_manifest_load(data, len(data), h, err, len(err)))


def decode_bpk_manifest(data: bytes) -> BpkModelManifest:
    """decode_bpk_manifest (import.rs:460-498): the container form only."""
    data = bytes(data)
    if len(data) >= 8 and not data.startswith(BPK_MAGIC):
        raise _abi.InvalidFormat("invalid model format: missing bpk magic")
    if len(data) < BPK_HEADER_LEN:
        raise _abi.InvalidFormat("invalid model format: bpk file is shorter than header: "
                                 f"{len(data)} < {BPK_HEADER_LEN}")
    return load_manifest_bytes(data)


def load_manifest(path) -> BpkModelManifest:
    """load_manifest (import.rs:378-381)."""
    p = str(path).encode()
    return _load(lambda h, err: lib().npa_manifest_load_file(p, h, err, len(err)))


def encode_bpk_manifest(payload: bytes) -> bytes:
    """encode_bpk_manifest (import.rs:444-458) for a serialized JSON payload."""
    payload = bytes(payload)
    L = lib()
    need = C.c_size_t()
    _check(L.npa_bpk_encode(payload, len(payload), None, 0, C.byref(need)))
    out = C.create_string_buffer(need.value)
    _check(L.npa_bpk_encode(payload, len(payload), out, need.value, C.byref(need)))
    return out.raw[:need.value]


def sha256(data: bytes) -> bytes:
    data = bytes(data)
    out = C.create_string_buffer(32)
    _check(lib().npa_sha256(data, len(data), out))
    return out.raw
