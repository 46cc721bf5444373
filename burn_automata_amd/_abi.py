"""ctypes mirror of ``include/npa_abi.h`` (plain-data structs, status codes, errors).

The status codes map 1:1 onto ``KernelError`` of the reference
(crates/burn_automata_kernels/src/config.rs:101-137); :func:`check` raises the
matching Python exception class so callers see the reference's error variants.
"""
from __future__ import annotations

import ctypes as C

u32 = C.c_uint32
f32 = C.c_float

NPA_OK = 0
NPA_ERR_INVALID_DIM = 1
NPA_ERR_INVALID_EPS = 2
NPA_ERR_INVALID_GRID_SIZE = 3
NPA_ERR_PARTICLE_MODE_POW2 = 4
NPA_ERR_POSITION_SHAPE = 10
NPA_ERR_STATE_SHAPE = 11
NPA_ERR_OUTPUT_SHAPE = 12
NPA_ERR_INVALID_ARGUMENT = 13
NPA_ERR_INVALID_MODEL = 20
NPA_ERR_IO = 21
NPA_ERR_JSON = 22
NPA_ERR_INVALID_FORMAT = 23
NPA_ERR_DEVICE = 30
NPA_ERR_OUT_OF_MEMORY = 31
NPA_ERR_COORD_OVERFLOW = 32

# update-MLP engines (npa_context_set_mlp_engine / npa_state_set_mlp_engine)
MLP_VALU = 0
MLP_MFMA = 1
MLP_MFMA_BF16 = 2

# kernel ids for npa_profile_read
KERNEL_NAMES = ("hash_rank", "table_scan", "offsets_scan", "scatter", "density", "perceive", "splat",
                "mlp", "split", "active", "render", "raster")


class NpaGridCfg(C.Structure):
    _fields_ = [("dim", u32), ("boundary", u32), ("mode", u32), ("grid_size", u32 * 3),
                ("eps", f32), ("max_particles_per_block", u32)]


class NpaPerceptionOpts(C.Structure):
    _fields_ = [("state_grad", u32), ("density_grad", u32), ("eps0", f32),
                ("scale_equivariance", u32), ("particle_density_equivariance", u32),
                ("log_norm_grad", u32), ("log_norm_density_grad", u32),
                ("hybrid_state_gradient", u32), ("position_features", u32)]


class NpaModelCfg(C.Structure):
    _fields_ = [("spatial_dims", u32), ("state_dims", u32), ("hidden_dims", u32),
                ("eps0", f32), ("alpha", f32), ("density_grad", u32), ("state_grad", u32),
                ("log_norm_grad", u32), ("log_norm_density_grad", u32),
                ("equivariance", u32), ("position_features", u32)]


class NpaWeightsC(C.Structure):
    _fields_ = [("w1", C.c_void_p), ("b1", C.c_void_p), ("w2", C.c_void_p), ("b2", C.c_void_p)]


class NpaGaussianDecodeCfg(C.Structure):
    _fields_ = [("mode", u32), ("sigma", f32), ("min_scale", f32), ("max_scale", f32),
                ("max_anisotropy", f32), ("opacity_scale", f32), ("min_opacity", f32),
                ("max_opacity", f32), ("sh_degree", u32)]


class NpaSplat2dCfg(C.Structure):
    _fields_ = [("image_size", u32), ("sigma", f32), ("lo", f32), ("hi", f32),
                ("normalize_color", u32), ("y_up", u32), ("pixel_size", f32)]


class NpaRenderCfg(C.Structure):
    _fields_ = [("image_size", u32), ("sigma", f32), ("min_sigma", f32), ("max_sigma", f32),
                ("gaussian_decode_mode", u32), ("world_scale", f32), ("target_samples", u32),
                ("opacity_logit_bias", f32), ("density_weight", f32), ("color_weight", f32),
                ("depth_weight", f32)]


class NpaRasterCamera(C.Structure):
    _fields_ = [("view", f32 * 16), ("fx", f32), ("fy", f32), ("cx", f32), ("cy", f32),
                ("width", u32), ("height", u32), ("near_plane", f32), ("far_plane", f32),
                ("sh_degree", u32), ("color_mode", u32)]


class KernelError(RuntimeError):
    """Base of the KernelError variants (config.rs:101-137)."""

    code = -1

    def __init__(self, message: str = ""):
        super().__init__(message)
        self.message = message


class InvalidDim(KernelError):
    code = NPA_ERR_INVALID_DIM


class InvalidEps(KernelError):
    code = NPA_ERR_INVALID_EPS


class InvalidGridSize(KernelError):
    code = NPA_ERR_INVALID_GRID_SIZE


class ParticleModeRequiresPowerOfTwo(KernelError):
    code = NPA_ERR_PARTICLE_MODE_POW2


class PositionShape(KernelError):
    code = NPA_ERR_POSITION_SHAPE


class StateShape(KernelError):
    code = NPA_ERR_STATE_SHAPE


class OutputShape(KernelError):
    code = NPA_ERR_OUTPUT_SHAPE


class InvalidArgument(KernelError):
    code = NPA_ERR_INVALID_ARGUMENT


class InvalidModel(KernelError):
    """AutomataError::InvalidModel (crates/burn_automata/src/error.rs)."""

    code = NPA_ERR_INVALID_MODEL


class IoError(KernelError):
    """AutomataError::Io."""

    code = NPA_ERR_IO


class JsonError(KernelError):
    """AutomataError::Json (a manifest that is not the reference's JSON)."""

    code = NPA_ERR_JSON


class InvalidFormat(KernelError):
    """AutomataError::InvalidFormat (a damaged .bpk container)."""

    code = NPA_ERR_INVALID_FORMAT


class NpaManifestInfo(C.Structure):
    _fields_ = [("format_version", u32), ("model_kind", C.c_char_p), ("source", C.c_char_p),
                ("auxiliary_input_dims", u32), ("decoder_dims", C.c_int64),
                ("output_dims", C.c_int64), ("stopgrad_pos", u32), ("stopgrad_state", u32),
                ("initialization_particles", u32)]


class DeviceError(KernelError):
    code = NPA_ERR_DEVICE


class OutOfMemory(KernelError):
    code = NPA_ERR_OUT_OF_MEMORY


class CoordOverflow(KernelError):
    code = NPA_ERR_COORD_OVERFLOW


_BY_CODE = {cls.code: cls for cls in (
    InvalidDim, InvalidEps, InvalidGridSize, ParticleModeRequiresPowerOfTwo, PositionShape,
    StateShape, OutputShape, InvalidArgument, InvalidModel, IoError, JsonError, InvalidFormat,
    DeviceError, OutOfMemory, CoordOverflow)}


def error_for(code: int, message: str = "") -> KernelError:
    cls = _BY_CODE.get(int(code), KernelError)
    err = cls(message or f"npa status {code}")
    if cls is KernelError:
        err.code = int(code)
    return err
