"""Loads libnpa_hip.so (built in-tree by ``burn_automata_amd.build``) and declares its C ABI.

There is no fallback: when the library is missing the import fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

from . import _abi

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnpa_hip.so")
_lib = None

P = C.c_void_p
u32 = C.c_uint32
u64 = C.c_uint64
f32 = C.c_float
sz = C.c_size_t
st = C.c_int


def _decl(L):
    ptr = C.POINTER
    L.npa_version.argtypes = []
    L.npa_version.restype = C.c_char_p
    L.npa_context_create.argtypes = [C.c_int, P, ptr(P)]
    L.npa_context_destroy.argtypes = [P]
    L.npa_context_destroy.restype = None
    L.npa_context_set_stream.argtypes = [P, P]
    L.npa_context_set_host_io.argtypes = [P, C.c_int]
    L.npa_context_synchronize.argtypes = [P]
    L.npa_last_error.argtypes = [P]
    L.npa_last_error.restype = C.c_char_p
    L.npa_build_hashgrid.argtypes = [P, P, u32, u32, ptr(_abi.NpaGridCfg), P, sz, P, P, sz]
    L.npa_neighbor_lists.argtypes = [P, P, u32, u32, ptr(_abi.NpaGridCfg), P, P, sz, ptr(sz)]
    L.npa_perceive.argtypes = [P, P, P, u32, u32, u32, ptr(_abi.NpaGridCfg),
                               ptr(_abi.NpaPerceptionOpts), P, sz, P, P, P, P, ptr(u32)]
    L.npa_mlp_forward.argtypes = [P, P, u32, ptr(_abi.NpaModelCfg), ptr(_abi.NpaWeightsC), f32, P,
                                  P]
    L.npa_euler_step.argtypes = [P, P, P, P, P, u32, u32, u32, ptr(_abi.NpaGridCfg), f32, P, P, P]
    L.npa_step.argtypes = [P, P, P, u32, u32, ptr(_abi.NpaGridCfg), ptr(_abi.NpaModelCfg),
                           ptr(_abi.NpaWeightsC), f32, P, P, P, P]
    L.npa_step_noalloc.argtypes = [P, P, P, u32, u32, ptr(_abi.NpaGridCfg), ptr(_abi.NpaModelCfg),
                                   ptr(_abi.NpaWeightsC), f32, P, P, P, P]
    L.npa_update_mask.argtypes = [P, u32, u32, f32, u32, u64, P]
    L.npa_decode_gaussians_3d.argtypes = [P, P, P, u32, u32, ptr(_abi.NpaGaussianDecodeCfg), P, P,
                                          P, P]
    L.npa_splat_2d.argtypes = [P, P, P, u32, ptr(_abi.NpaSplat2dCfg), P]
    L.npa_splat_2d_tiled.argtypes = [P, P, P, u32, u32, ptr(_abi.NpaSplat2dCfg), u32, P]
    L.npa_perceive_adjoint.argtypes = [P, P, P, u32, u32, u32, ptr(_abi.NpaGridCfg),
                                       ptr(_abi.NpaPerceptionOpts), P, sz, P, P]
    L.npa_render_views.argtypes = [P, P, P, P, P, u32, P, u32, ptr(_abi.NpaRenderCfg), P]
    L.npa_render_attributes.argtypes = [P, P, u32, u32, ptr(_abi.NpaRenderCfg), P, P, P, P]
    L.npa_state_render_views.argtypes = [P, P, u32, ptr(_abi.NpaRenderCfg), P]
    L.npa_raster_gaussians_3d.argtypes = [P, P, P, P, P, u32, ptr(_abi.NpaRasterCamera), P]
    L.npa_state_raster_gaussians_3d.argtypes = [P, ptr(_abi.NpaGaussianDecodeCfg),
                                                ptr(_abi.NpaRasterCamera), P]
    L.npa_manifest_load.argtypes = [P, sz, ptr(P), C.c_char_p, sz]
    L.npa_manifest_load_file.argtypes = [C.c_char_p, ptr(P), C.c_char_p, sz]
    L.npa_manifest_destroy.argtypes = [P]
    L.npa_manifest_destroy.restype = None
    L.npa_manifest_info.argtypes = [P, ptr(_abi.NpaManifestInfo)]
    L.npa_manifest_model.argtypes = [P, ptr(_abi.NpaModelCfg), ptr(_abi.NpaGridCfg), ptr(_abi.NpaWeightsC)]
    L.npa_manifest_initialization.argtypes = [P, ptr(P), ptr(P), ptr(u32)]
    L.npa_bpk_encode.argtypes = [P, sz, P, sz, ptr(sz)]
    L.npa_sha256.argtypes = [P, sz, P]
    L.npa_context_set_mlp_engine.argtypes = [P, C.c_int]
    L.npa_state_set_mlp_engine.argtypes = [P, C.c_int]
    L.npa_state_create.argtypes = [P, ptr(_abi.NpaModelCfg), ptr(_abi.NpaWeightsC),
                                   ptr(_abi.NpaGridCfg), P, P, u32, u32, f32, f32, u64, ptr(P)]
    L.npa_state_destroy.argtypes = [P]
    L.npa_state_destroy.restype = None
    L.npa_state_step.argtypes = [P, u32]
    L.npa_state_read.argtypes = [P, P, P, P]
    L.npa_state_update_model.argtypes = [P, ptr(_abi.NpaWeightsC)]
    L.npa_state_step_index.argtypes = [P, ptr(u64)]
    L.npa_state_buffers.argtypes = [P, ptr(P), ptr(P)]
    L.npa_state_splat_2d.argtypes = [P, ptr(_abi.NpaSplat2dCfg), P]
    L.npa_state_splat_2d_tiled.argtypes = [P, ptr(_abi.NpaSplat2dCfg), u32, P]
    L.npa_state_decode_gaussians_3d.argtypes = [P, ptr(_abi.NpaGaussianDecodeCfg), P, P, P, P]
    L.npa_state_write_gaussians.argtypes = [P, u32, P, P, P, P]
    L.npa_state_step_into_gaussians.argtypes = [P, u32, u32, P, P, P, P]
    L.npa_profile_enable.argtypes = [P, C.c_int]
    L.npa_profile_reset.argtypes = [P]
    L.npa_profile_read.argtypes = [P, C.c_int, ptr(C.c_double), ptr(u64)]
    L.npa_state_pair_counts.argtypes = [P, ptr(u64), ptr(u64), ptr(u64), ptr(u64), ptr(u64)]
    for name in ("npa_context_create", "npa_context_set_stream", "npa_context_set_host_io",
                 "npa_context_synchronize", "npa_build_hashgrid", "npa_neighbor_lists",
                 "npa_perceive", "npa_mlp_forward", "npa_euler_step", "npa_step",
                 "npa_update_mask", "npa_decode_gaussians_3d", "npa_splat_2d", "npa_state_create",
                 "npa_state_step", "npa_state_read", "npa_state_update_model",
                 "npa_state_step_index", "npa_state_buffers", "npa_state_splat_2d",
                 "npa_state_decode_gaussians_3d", "npa_profile_enable", "npa_profile_reset",
                 "npa_profile_read", "npa_state_pair_counts", "npa_splat_2d_tiled",
                 "npa_state_splat_2d_tiled", "npa_context_set_mlp_engine",
                 "npa_state_set_mlp_engine", "npa_manifest_load", "npa_manifest_load_file",
                 "npa_manifest_info", "npa_manifest_model", "npa_manifest_initialization",
                 "npa_bpk_encode", "npa_sha256", "npa_render_views", "npa_render_attributes",
                 "npa_state_render_views", "npa_perceive_adjoint", "npa_raster_gaussians_3d",
                 "npa_state_raster_gaussians_3d", "npa_step_noalloc", "npa_state_write_gaussians",
                 "npa_state_step_into_gaussians"):
        getattr(L, name).restype = st


EXPORTED = (
    "npa_context_create", "npa_context_destroy", "npa_context_set_stream", "npa_context_set_host_io",
    "npa_context_synchronize", "npa_last_error", "npa_version", "npa_build_hashgrid",
    "npa_neighbor_lists", "npa_perceive", "npa_mlp_forward", "npa_euler_step", "npa_step",
    "npa_update_mask", "npa_decode_gaussians_3d", "npa_splat_2d", "npa_state_create",
    "npa_state_destroy", "npa_state_step", "npa_state_read", "npa_state_update_model",
    "npa_state_step_index", "npa_state_buffers", "npa_state_splat_2d",
    "npa_state_decode_gaussians_3d", "npa_profile_enable", "npa_profile_reset", "npa_profile_read",
    "npa_state_pair_counts", "npa_splat_2d_tiled", "npa_state_splat_2d_tiled",
    "npa_context_set_mlp_engine", "npa_state_set_mlp_engine", "npa_manifest_load",
    "npa_manifest_load_file", "npa_manifest_destroy", "npa_manifest_info", "npa_manifest_model",
    "npa_manifest_initialization", "npa_bpk_encode", "npa_sha256", "npa_render_views",
    "npa_render_attributes", "npa_state_render_views", "npa_perceive_adjoint",
    "npa_raster_gaussians_3d", "npa_state_raster_gaussians_3d", "npa_step_noalloc", "npa_state_write_gaussians",
    "npa_state_step_into_gaussians")


def lib():
    """The loaded library (raises ImportError when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m burn_automata_amd.build` "
                "(the HIP path has no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        _decl(L)
        _lib = L
    return _lib
