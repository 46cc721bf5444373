"""`.bpk` model files through libnpa_hip.so's loader (host code; runs without a GPU).

Mirrors the reference's tests in crates/burn_automata/tests/core/import_bridge.rs:4-95 (manifest
round trips, corruption rejected by the checksum, parameter count of the PyTorch import fixture)
and pins the container format of import.rs:16-18, 444-498 with an independent encoder written
here (struct + hashlib), the JSON rules serde_json applies to the manifest types, and SHA-256
against hashlib.
"""
import hashlib
import json
import struct

import numpy as np
import pytest

from burn_automata_amd import _abi
from burn_automata_amd import bpk
from burn_automata_amd import synthetic as syn
from burn_automata_amd.config import Boundary, EquivarianceMode, HashGridConfig, HashGridMode, NpaConfig


def f32_text(x) -> str:
    """The shortest decimal that reads back as the same f32 (how serde_json writes an f32)."""
    return repr(np.float32(x)).replace("np.float32(", "").rstrip(")")


def manifest_json(model: NpaConfig, grid: HashGridConfig, weights, source="unit-test",
                  initialization=None, drop=(), extra=None, config_extra=None) -> bytes:
    """BpkModelManifest as serde_json::to_vec writes it: compact, fields in declaration order."""
    def arr(a):
        return "[" + ",".join(f32_text(v) for v in np.asarray(a, np.float32).ravel()) + "]"

    eq = {EquivarianceMode.NoEquivariance: "None", EquivarianceMode.ParticleDensity: "ParticleDensity",
          EquivarianceMode.ParticleDensityAndScale: "ParticleDensityAndScale"}[model.equivariance]
    cfg = [("spatial_dims", str(model.spatial_dims)), ("state_dims", str(model.state_dims)),
           ("hidden_dims", str(model.hidden_dims)), ("eps0", f32_text(model.eps0)),
           ("alpha", f32_text(model.alpha)), ("density_grad", json.dumps(model.density_grad)),
           ("state_grad", json.dumps(model.state_grad)), ("log_norm_grad", json.dumps(model.log_norm_grad)),
           ("log_norm_density_grad", json.dumps(model.log_norm_density_grad)),
           ("stopgrad_pos", "true"), ("stopgrad_state", "false"), ("equivariance", json.dumps(eq)),
           ("position_features", json.dumps(model.position_features)), ("auxiliary_input_dims", "0"),
           ("decoder_dims", "null"), ("output_dims", "null")] + list((config_extra or {}).items())
    hg = [("dim", str(grid.dim)), ("boundary", json.dumps(Boundary(grid.boundary).name)),
          ("mode", json.dumps(HashGridMode(grid.mode).name)),
          ("grid_size", "[" + ",".join(str(int(v)) for v in grid.grid_size) + "]"),
          ("eps", f32_text(grid.eps)), ("max_particles_per_block", str(grid.max_particles_per_block))]
    w = [(k, arr(weights[k])) for k in ("w1", "b1", "w2", "b2")]
    top = [("format_version", "1"), ("model_kind", '"npa"'),
           ("source", json.dumps(source) if source is not None else "null"),
           ("config", "{" + ",".join(f'"{k}":{v}' for k, v in cfg if k not in drop) + "}"),
           ("hashgrid", "{" + ",".join(f'"{k}":{v}' for k, v in hg if k not in drop) + "}"),
           ("weights", "{" + ",".join(f'"{k}":{v}' for k, v in w if k not in drop) + "}")]
    if initialization is not None:
        pos, st = initialization
        top.append(("initialization",
                    '{"positions":[' + ",".join(arr(p) for p in np.asarray(pos, np.float32)) +
                    '],"states":' + arr(st) + "}"))
    top += list((extra or {}).items())
    return ("{" + ",".join(f'"{k}":{v}' for k, v in top if k not in drop) + "}").encode()


def as_f32(cfg):
    """A config with its float fields rounded to f32, as the reference holds them."""
    if isinstance(cfg, NpaConfig):
        return cfg.replace(eps0=float(np.float32(cfg.eps0)), alpha=float(np.float32(cfg.alpha)))
    return cfg.replace(eps=float(np.float32(cfg.eps)))


def container(payload: bytes, version: int = 1) -> bytes:
    """The container layout of encode_bpk_manifest (import.rs:444-458), written independently."""
    return b"BAUTBPK1" + struct.pack("<IQ", version, len(payload)) + hashlib.sha256(payload).digest() + payload


@pytest.fixture(scope="module")
def c1():
    w = syn.workload("c1", particles=64)
    return w["model"], w["grid"], w["weights"]


def test_sha256_matches_hashlib():
    rng = np.random.default_rng(0)
    for n in list(range(0, 200)) + [1000, 4096, 1 << 20]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert bpk.sha256(data) == hashlib.sha256(data).digest(), n


def test_encode_matches_the_container_layout(c1):
    m, g, w = c1
    payload = manifest_json(m, g, w)
    assert bpk.encode_bpk_manifest(payload) == container(payload)


def test_json_manifest_roundtrips_seeded_model(c1):
    """manifest_roundtrips_seeded_model (import_bridge.rs:4-18)."""
    m, g, w = c1
    got = bpk.load_manifest_bytes(manifest_json(m, g, w))
    assert got.format_version == 1 and got.model_kind == "npa" and got.source == "unit-test"
    assert got.config == as_f32(m) and got.hashgrid == as_f32(g)
    for k in ("w1", "b1", "w2", "b2"):
        np.testing.assert_array_equal(got.weights[k], w[k])
    assert got.initialization is None and got.decoder_dims is None


def test_bpk_roundtrips_and_rejects_corruption(c1, tmp_path):
    """bpk_manifest_roundtrips_and_rejects_corruption (import_bridge.rs:21-42)."""
    m, g, w = c1
    data = container(manifest_json(m, g, w))
    path = tmp_path / "manifest_roundtrip.bpk"
    path.write_bytes(data)
    got = bpk.load_manifest(path)
    assert got.config == as_f32(m)
    np.testing.assert_array_equal(got.weights["w1"], w["w1"])
    bad = bytearray(data)
    bad[-5] ^= 0x01
    with pytest.raises(_abi.InvalidFormat, match="checksum"):
        bpk.decode_bpk_manifest(bytes(bad))
    with pytest.raises(_abi.IoError):
        bpk.load_manifest(tmp_path / "missing.bpk")


def test_container_header_errors(c1):
    """decode_bpk_manifest's checks, in the reference's order (import.rs:460-498)."""
    m, g, w = c1
    payload = manifest_json(m, g, w)
    with pytest.raises(_abi.InvalidFormat, match="shorter than header: 20 < 52"):
        bpk.load_manifest_bytes(container(payload)[:20])
    with pytest.raises(_abi.InvalidFormat, match="unsupported bpk container version 2"):
        bpk.load_manifest_bytes(container(payload, version=2))
    with pytest.raises(_abi.InvalidFormat, match="payload length mismatch"):
        bpk.load_manifest_bytes(container(payload) + b" ")
    with pytest.raises(_abi.InvalidFormat, match="missing bpk magic"):
        bpk.decode_bpk_manifest(payload)


def test_serde_json_rules(c1):
    m, g, w = c1
    # unknown fields are ignored; serde defaults fill absent fields
    got = bpk.load_manifest_bytes(manifest_json(m, g, w, extra={"future": '{"x":[1,2,{"y":null}]}'},
                                                config_extra={"note": '"ok"'}))
    assert got.config == as_f32(m)
    no_defaults = manifest_json(m, g, w, drop=("equivariance", "position_features", "auxiliary_input_dims",
                                               "decoder_dims", "output_dims", "source"))
    got = bpk.load_manifest_bytes(no_defaults)
    assert got.config.equivariance == EquivarianceMode.ParticleDensityAndScale
    assert got.config.position_features is False and got.source is None
    # required fields, types and variants
    with pytest.raises(_abi.JsonError, match="missing field `stopgrad_pos`"):
        bpk.load_manifest_bytes(manifest_json(m, g, w, drop=("stopgrad_pos",)))
    with pytest.raises(_abi.JsonError, match="missing field `w2`"):
        bpk.load_manifest_bytes(manifest_json(m, g, w, drop=("w2",)))
    with pytest.raises(_abi.JsonError, match="unknown variant"):
        bpk.load_manifest_bytes(manifest_json(m, g, w).replace(b'"Clamped"', b'"Clampd"'))
    with pytest.raises(_abi.JsonError, match="unsigned integer"):
        bpk.load_manifest_bytes(manifest_json(m, g, w).replace(b'"hidden_dims":128', b'"hidden_dims":128.0'))
    with pytest.raises(_abi.JsonError):
        bpk.load_manifest_bytes(manifest_json(m, g, w)[:-1])
    # usize fields the C ABI carries as u32 are refused above u32::MAX instead of truncated
    # (2^32 + 64 would otherwise read as 64 and pass validation)
    big = manifest_json(m, g, w).replace(b'"grid_size":[64,64,1]', b'"grid_size":[4294967360,64,1]')
    assert big != manifest_json(m, g, w)
    with pytest.raises(_abi.JsonError, match="out of range for u32"):
        bpk.load_manifest_bytes(big)
    with pytest.raises(_abi.JsonError, match="out of range for u32"):
        bpk.load_manifest_bytes(manifest_json(m, g, w).replace(b'"state_dims":16', b'"state_dims":4294967312'))
    # f32 fields: shortest f32 text and the f64 text of the same f32 read the same
    got = bpk.load_manifest_bytes(manifest_json(m, g, w).replace(b'"eps":0.05', b'"eps":0.05000000074505806'))
    assert got.hashgrid.eps == np.float32(0.05)


def test_model_validation(c1):
    """validate_manifest (import.rs:500-506): NpaModel::validate and the weight lengths."""
    m, g, w = c1
    bad = dict(w, w1=w["w1"][:-1])
    with pytest.raises(_abi.InvalidModel, match=f"w1 len {w['w1'].size - 1} != {w['w1'].size}"):
        bpk.load_manifest_bytes(manifest_json(m, g, bad))
    with pytest.raises(_abi.InvalidModel, match="spatial_dims must be 2 or 3, got 4"):
        bpk.load_manifest_bytes(manifest_json(m.replace(spatial_dims=4), g, w))


def test_pytorch_fixture_parameter_count():
    """pytorch_npa_checkpoint_imports_to_bpk (import_bridge.rs:73-95): a 2D model with one state
    channel and two hidden units has 23 parameters."""
    m = NpaConfig(spatial_dims=2, state_dims=1, hidden_dims=2, eps0=0.1)
    g = HashGridConfig(2, Boundary.Clamped, HashGridMode.Particle, (64, 64, 1), 0.1, 32)
    w = syn.seeded_weights(m, 3)
    got = bpk.load_manifest_bytes(container(manifest_json(m, g, w)))
    assert sum(v.size for v in got.weights.values()) == 23
    assert got.hashgrid.eps == np.float32(0.1) and got.hashgrid.grid_size == (64, 64, 1)


def test_initialization_roundtrip_and_checks(c1):
    m, g, w = c1
    pos = syn.uniform_disk(10, 3)
    st = syn.normal_states(10, m.state_dims, 3)
    got = bpk.load_manifest_bytes(container(manifest_json(m, g, w, initialization=(pos, st))))
    np.testing.assert_array_equal(got.initialization[0], pos)
    np.testing.assert_array_equal(got.initialization[1], st.ravel())
    with pytest.raises(_abi.InvalidModel, match="cannot be empty"):
        bpk.load_manifest_bytes(manifest_json(m, g, w, initialization=(np.zeros((0, 4)), np.zeros(0))))
    with pytest.raises(_abi.InvalidModel, match="state values; expected 10 positions"):
        bpk.load_manifest_bytes(manifest_json(m, g, w, initialization=(pos, st.ravel()[:-1])))
