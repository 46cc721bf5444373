"""MI355X-native fixed-NPA rollout: hand-written gfx950 HIP kernels behind a C ABI.

The hot path of mosure/burn_automata - hashgrid build, SPH perception, update MLP,
masked residual update and Gaussian decode - as libnpa_hip.so (include/npa_abi.h),
with this package as the host-side mirror of the reference's operator surface.
"""
from .config import (Boundary, EquivarianceMode, GaussianDecodeConfig, GaussianDecodeMode,
                     HashGridConfig, HashGridMode, NpaConfig, PerceptionOptions, RolloutConfig,
                     Splat2dConfig)

__all__ = [
    "Boundary", "EquivarianceMode", "GaussianDecodeConfig", "GaussianDecodeMode", "HashGridConfig",
    "HashGridMode", "NpaConfig", "PerceptionOptions", "RolloutConfig", "Splat2dConfig",
]
