"""CPU checks of the C-ABI boundary (include/npa_abi.h <-> libnpa_hip.so <-> the ctypes mirror).

No compute call runs here (there is no GPU in this container): the checks cover the exported
symbol set, the prototypes' arity against the Python declarations, the struct layouts against
the C compiler's, the status codes, and the error a context reports without a device.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

import pytest

from burn_automata_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "npa_abi.h")


def _header_text():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _prototypes():
    """name -> parameter list of every function the header declares."""
    out = {}
    for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(npa_\w+)\s*\(([^)]*)\)\s*;", _header_text(), re.M):
        params = " ".join(m.group(2).split())
        out[m.group(1)] = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
    return out


@pytest.fixture(scope="module")
def lib():
    from burn_automata_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from burn_automata_amd import build
        build.build()
    return _lib


def test_header_declares_the_operator_surface():
    names = set(_prototypes())
    for want in ("npa_build_hashgrid", "npa_neighbor_lists", "npa_perceive", "npa_mlp_forward",
                 "npa_euler_step", "npa_step", "npa_update_mask", "npa_decode_gaussians_3d",
                 "npa_splat_2d", "npa_state_create", "npa_state_step", "npa_state_read",
                 "npa_state_update_model", "npa_state_destroy", "npa_last_error"):
        assert want in names


def test_library_exports_every_declared_symbol(lib):
    nm = subprocess.run(["nm", "-D", "--defined-only", lib.LIB_PATH], check=True,
                        stdout=subprocess.PIPE, text=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line}
    declared = set(_prototypes())
    assert declared <= exported, sorted(declared - exported)
    assert set(lib.EXPORTED) == declared


def test_ctypes_declarations_match_prototype_arity(lib):
    L = lib.lib()
    for name, params in _prototypes().items():
        fn = getattr(L, name)
        assert fn.argtypes is not None and len(fn.argtypes) == len(params), (name, params)


def test_status_codes_match_header():
    text = _header_text()
    codes = {m.group(1): int(m.group(2)) for m in re.finditer(r"\b(NPA_(?:OK|ERR_\w+))\s*=\s*(\d+)", text)}
    assert len(codes) == 16
    for name, value in codes.items():
        assert getattr(_abi, name) == value, name
        if name != "NPA_OK":
            assert type(_abi.error_for(value)).code == value


def test_struct_layouts_match_the_c_compiler(tmp_path):
    structs = {
        "npa_grid_cfg": _abi.NpaGridCfg, "npa_perception_opts": _abi.NpaPerceptionOpts,
        "npa_model_cfg": _abi.NpaModelCfg, "npa_weights": _abi.NpaWeightsC,
        "npa_gaussian_decode_cfg": _abi.NpaGaussianDecodeCfg, "npa_splat2d_cfg": _abi.NpaSplat2dCfg,
        "npa_manifest_info_t": _abi.NpaManifestInfo,
    }
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "npa_abi.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), "-o", str(exe), str(src)],
                   check=True)
    got = subprocess.run([str(exe)], check=True, stdout=subprocess.PIPE, text=True).stdout.split("\n")
    for line in filter(None, got):
        cname, what, value = line.split()
        py = structs[cname]
        want = C.sizeof(py) if what == "size" else getattr(py, what).offset
        assert int(value) == want, line


def test_version_and_missing_device_error(lib):
    L = lib.lib()
    assert L.npa_version().startswith(b"npa_hip")
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a device is present")
    except ImportError:
        pass
    ctx = C.c_void_p()
    assert L.npa_context_create(0, None, C.byref(ctx)) == _abi.NPA_ERR_DEVICE
    assert not ctx.value


def test_missing_library_fails_loudly(monkeypatch):
    from burn_automata_amd import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", os.path.join(ROOT, "does_not_exist.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError, match="no CPU fallback"):
        _lib.lib()


def test_log1pf_matches_host_libm_for_every_float(tmp_path):
    """burn_automata_amd/csrc/npa_math.hpp (the device log1pf) against the host libm's log1pf
    for every float in [-1, +inf] - the reference's ln_1p on Linux."""
    exe = tmp_path / "check_log1p"
    subprocess.run(["g++", "-O2", "-std=c++17", "-fopenmp", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(ROOT, "tests", "native", "check_log1p.cpp")], check=True)
    for lo, hi in (("0x00000000", "0x7f800000"), ("0x80000000", "0xbf800000")):
        r = subprocess.run([str(exe), lo, hi], stdout=subprocess.PIPE, text=True, timeout=600)
        assert r.returncode == 0 and "mismatches 0" in r.stdout, r.stdout
