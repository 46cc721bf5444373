"""Configuration types mirroring the reference's Rust structs and presets.

* ``HashGridConfig`` / ``Boundary`` / ``HashGridMode``:
  crates/burn_automata_kernels/src/config.rs:4-99
* ``PerceptionOptions``: crates/burn_automata_kernels/src/reference/types.rs:4-31
* ``NpaConfig`` / ``EquivarianceMode``: crates/burn_automata/src/config.rs:22-199
* ``GaussianDecodeConfig`` / ``GaussianDecodeMode``: crates/burn_automata_kernels/src/gaussian.rs:13-51
* ``Splat2dConfig``: crates/burn_automata_kernels/src/splat.rs:6-28
* ``RenderLossConfig`` / ``RenderViewPreset``: crates/burn_automata/src/render_loss.rs:25-63
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass, field
from enum import IntEnum

from . import _abi


class Boundary(IntEnum):
    Periodic = 0
    Clamped = 1


class HashGridMode(IntEnum):
    Grid = 0
    Particle = 1


class EquivarianceMode(IntEnum):
    NoEquivariance = 0
    ParticleDensity = 1
    ParticleDensityAndScale = 2


class GaussianDecodeMode(IntEnum):
    ParticlePoint = 0
    GaussianSh0FixedScale = 1
    GaussianSh0LearnedScale = 2
    GaussianSh0Oriented = 3


@dataclass
class HashGridConfig:
    dim: int = 2
    boundary: Boundary = Boundary.Clamped
    mode: HashGridMode = HashGridMode.Particle
    grid_size: tuple = (64, 64, 1)
    eps: float = 0.1
    max_particles_per_block: int = 32

    @staticmethod
    def growing_2d() -> "HashGridConfig":
        return HashGridConfig(2, Boundary.Clamped, HashGridMode.Particle, (64, 64, 1), 0.1, 32)

    @staticmethod
    def texture_2d() -> "HashGridConfig":
        return HashGridConfig(2, Boundary.Periodic, HashGridMode.Grid, (10, 10, 1), 0.2, 32)

    @staticmethod
    def growing_3dgs() -> "HashGridConfig":
        return HashGridConfig(3, Boundary.Clamped, HashGridMode.Particle, (32, 32, 32), 0.1, 64)

    def replace(self, **kw) -> "HashGridConfig":
        return dataclasses.replace(self, **kw)

    def cell_count(self) -> int:
        n = 1
        for a in range(self.dim):
            n *= int(self.grid_size[a])
        return n

    def spatial_mem_dims(self) -> int:
        return 4 if self.dim == 3 else 2

    def to_c(self) -> _abi.NpaGridCfg:
        c = _abi.NpaGridCfg()
        c.dim = int(self.dim)
        c.boundary = int(self.boundary)
        c.mode = int(self.mode)
        for a in range(3):
            c.grid_size[a] = int(self.grid_size[a])
        c.eps = float(self.eps)
        c.max_particles_per_block = int(self.max_particles_per_block)
        return c


@dataclass
class PerceptionOptions:
    state_grad: bool = True
    density_grad: bool = True
    eps0: float = 0.1
    scale_equivariance: bool = True
    particle_density_equivariance: bool = True
    log_norm_grad: bool = False
    log_norm_density_grad: bool = False
    hybrid_state_gradient: bool = True
    position_features: bool = False

    @staticmethod
    def new(state_grad: bool, density_grad: bool, eps0: float) -> "PerceptionOptions":
        """PerceptionOptions::new (types.rs:17-31)."""
        return PerceptionOptions(state_grad, density_grad, eps0)

    def feature_dims(self, state_dims: int, dim: int) -> int:
        return (state_dims * 2 + int(self.state_grad) * state_dims * dim
                + int(self.density_grad) * dim + int(self.position_features) * dim)

    def to_c(self) -> _abi.NpaPerceptionOpts:
        c = _abi.NpaPerceptionOpts()
        for f in ("state_grad", "density_grad", "scale_equivariance",
                  "particle_density_equivariance", "log_norm_grad", "log_norm_density_grad",
                  "hybrid_state_gradient", "position_features"):
            setattr(c, f, int(bool(getattr(self, f))))
        c.eps0 = float(self.eps0)
        return c


@dataclass
class NpaConfig:
    spatial_dims: int = 2
    state_dims: int = 16
    hidden_dims: int = 128
    eps0: float = 0.1
    alpha: float = 0.5
    density_grad: bool = True
    state_grad: bool = True
    log_norm_grad: bool = True
    log_norm_density_grad: bool = True
    equivariance: EquivarianceMode = EquivarianceMode.ParticleDensityAndScale
    position_features: bool = False

    @staticmethod
    def growing_2d() -> "NpaConfig":
        return NpaConfig()

    @staticmethod
    def texture_2d() -> "NpaConfig":
        return NpaConfig(eps0=0.2)

    @staticmethod
    def growing_3dgs() -> "NpaConfig":
        return NpaConfig(spatial_dims=3, state_dims=24, hidden_dims=256, eps0=0.1, alpha=1.0)

    @staticmethod
    def point_mnist() -> "NpaConfig":
        return NpaConfig(hidden_dims=256, alpha=1.0)

    @staticmethod
    def torus_field_3dgs() -> "NpaConfig":
        return dataclasses.replace(NpaConfig.growing_3dgs(), position_features=True)

    def replace(self, **kw) -> "NpaConfig":
        return dataclasses.replace(self, **kw)

    def perception_dims(self) -> int:
        """config.rs:133-139 (no auxiliary inputs on this path)."""
        return (self.state_dims * 2 + int(self.state_grad) * self.state_dims * self.spatial_dims
                + int(self.density_grad) * self.spatial_dims
                + int(self.position_features) * self.spatial_dims)

    def update_dims(self) -> int:
        return self.spatial_dims + self.state_dims

    def scale_equivariant(self) -> bool:
        return self.equivariance == EquivarianceMode.ParticleDensityAndScale

    def particle_density_equivariant(self) -> bool:
        return self.equivariance in (EquivarianceMode.ParticleDensity,
                                     EquivarianceMode.ParticleDensityAndScale)

    def motion_eps(self, grid_eps: float) -> float:
        return grid_eps if self.scale_equivariant() else self.eps0

    def perception_options(self) -> PerceptionOptions:
        """The options NpaModel::step_cpu passes (crates/burn_automata/src/model.rs:784-800)."""
        return PerceptionOptions(
            state_grad=self.state_grad, density_grad=self.density_grad, eps0=self.eps0,
            scale_equivariance=self.scale_equivariant(),
            particle_density_equivariance=self.particle_density_equivariant(),
            log_norm_grad=self.log_norm_grad, log_norm_density_grad=self.log_norm_density_grad,
            hybrid_state_gradient=True, position_features=self.position_features)

    @staticmethod
    def for_preset(preset: str):
        """NpaConfig::for_preset (config.rs:183-190)."""
        table = {
            "growing_2d": (NpaConfig.growing_2d(), HashGridConfig.growing_2d()),
            "texture_2d": (NpaConfig.texture_2d(), HashGridConfig.texture_2d()),
            "growing_3dgs": (NpaConfig.growing_3dgs(), HashGridConfig.growing_3dgs()),
            "point_mnist": (NpaConfig.point_mnist(), HashGridConfig.growing_2d()),
        }
        return table[preset]

    def to_c(self) -> _abi.NpaModelCfg:
        c = _abi.NpaModelCfg()
        c.spatial_dims = int(self.spatial_dims)
        c.state_dims = int(self.state_dims)
        c.hidden_dims = int(self.hidden_dims)
        c.eps0 = float(self.eps0)
        c.alpha = float(self.alpha)
        c.density_grad = int(bool(self.density_grad))
        c.state_grad = int(bool(self.state_grad))
        c.log_norm_grad = int(bool(self.log_norm_grad))
        c.log_norm_density_grad = int(bool(self.log_norm_density_grad))
        c.equivariance = int(self.equivariance)
        c.position_features = int(bool(self.position_features))
        return c


@dataclass
class GaussianDecodeConfig:
    mode: GaussianDecodeMode = GaussianDecodeMode.GaussianSh0FixedScale
    sigma: float = 0.02
    min_scale: float = 0.001
    max_scale: float = 0.08
    max_anisotropy: float = 0.1
    opacity_scale: float = 0.15
    min_opacity: float = 0.001
    max_opacity: float = 0.95
    sh_degree: int = 0

    def sh_coeffs(self) -> int:
        if self.mode == GaussianDecodeMode.GaussianSh0Oriented:
            return (self.sh_degree + 1) ** 2
        return 1

    def to_c(self) -> _abi.NpaGaussianDecodeCfg:
        c = _abi.NpaGaussianDecodeCfg()
        c.mode = int(self.mode)
        for f in ("sigma", "min_scale", "max_scale", "max_anisotropy", "opacity_scale",
                  "min_opacity", "max_opacity"):
            setattr(c, f, float(getattr(self, f)))
        c.sh_degree = int(self.sh_degree)
        return c


@dataclass
class Splat2dConfig:
    image_size: int = 128
    sigma: float = 1.0
    lo: float = -1.0
    hi: float = 1.0
    normalize_color: bool = True
    y_up: bool = True
    pixel_size: float = 2.0 / 128.0

    def to_c(self) -> _abi.NpaSplat2dCfg:
        c = _abi.NpaSplat2dCfg()
        c.image_size = int(self.image_size)
        c.sigma = float(self.sigma)
        c.lo = float(self.lo)
        c.hi = float(self.hi)
        c.normalize_color = int(bool(self.normalize_color))
        c.y_up = int(bool(self.y_up))
        c.pixel_size = float(self.pixel_size)
        return c


class RenderViewPreset(IntEnum):
    """RenderViewPreset (crates/burn_automata/src/render_loss.rs:25-31)."""

    Xy = 0
    Xz = 1
    Yz = 2
    Iso = 3


ALL_VIEWS = (RenderViewPreset.Xy, RenderViewPreset.Xz, RenderViewPreset.Yz, RenderViewPreset.Iso)


@dataclass
class RenderLossConfig:
    """RenderLossConfig (crates/burn_automata/src/render_loss.rs:33-63), reference defaults."""

    image_size: int = 64
    sigma: float = 2.5
    min_sigma: float = 0.75
    max_sigma: float = 5.0
    gaussian_decode_mode: GaussianDecodeMode = GaussianDecodeMode.GaussianSh0FixedScale
    world_scale: float = 1.25
    target_samples: int = 8192
    opacity_logit_bias: float = 0.0
    density_weight: float = 1.0
    color_weight: float = 1.0
    depth_weight: float = 1.0

    def replace(self, **kw) -> "RenderLossConfig":
        return dataclasses.replace(self, **kw)

    def to_c(self) -> _abi.NpaRenderCfg:
        c = _abi.NpaRenderCfg()
        c.image_size = int(self.image_size)
        c.sigma = float(self.sigma)
        c.min_sigma = float(self.min_sigma)
        c.max_sigma = float(self.max_sigma)
        c.gaussian_decode_mode = int(self.gaussian_decode_mode)
        c.world_scale = float(self.world_scale)
        c.target_samples = int(self.target_samples)
        c.opacity_logit_bias = float(self.opacity_logit_bias)
        c.density_weight = float(self.density_weight)
        c.color_weight = float(self.color_weight)
        c.depth_weight = float(self.depth_weight)
        return c


class RasterColor(IntEnum):
    """How the oriented Gaussian raster reads the coefficients (NPA_RASTER_COLOR_*)."""

    SphericalHarmonics = 0  # real SH of degree sh_degree at the view direction, + 0.5, floored at 0
    Rgb = 1                 # coefficient 0 is the colour (decode_gaussians_3d, gaussian.rs:133-157)


@dataclass
class RasterCamera:
    """The camera of the oriented Gaussian raster (npa_raster_camera): a row-major world-to-camera
    matrix (camera looks down -z, +y up), pinhole intrinsics in pixels (y down), clip planes."""

    view: tuple
    fx: float
    fy: float
    cx: float
    cy: float
    width: int
    height: int
    near_plane: float = 0.1
    far_plane: float = 1000.0
    sh_degree: int = 0
    color_mode: RasterColor = RasterColor.SphericalHarmonics

    @classmethod
    def look_at(cls, eye, target=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0), width: int = 128, height: int = 128,
                fov_y: float = math.pi / 4, near_plane: float = 0.1, far_plane: float = 1000.0,
                sh_degree: int = 0, color_mode: RasterColor = RasterColor.SphericalHarmonics) -> "RasterCamera":
        """A camera at `eye` looking at `target` (bevy's Transform::looking_at with the default
        PerspectiveProjection: vertical field of view pi/4, near 0.1, far 1000), as the reference's
        headless raster test places it (crates/bevy_automata/tests/gaussian_gpu_link/headless.rs:23-27)."""
        eye = [float(v) for v in eye]
        back = [eye[k] - float(target[k]) for k in range(3)]
        nb = math.sqrt(sum(v * v for v in back))
        back = [v / nb for v in back]
        right = [up[1] * back[2] - up[2] * back[1], up[2] * back[0] - up[0] * back[2],
                 up[0] * back[1] - up[1] * back[0]]
        nr = math.sqrt(sum(v * v for v in right))
        right = [v / nr for v in right]
        upv = [back[1] * right[2] - back[2] * right[1], back[2] * right[0] - back[0] * right[2],
               back[0] * right[1] - back[1] * right[0]]
        view = []
        for row in (right, upv, back):
            view += row + [-sum(row[k] * eye[k] for k in range(3))]
        view += [0.0, 0.0, 0.0, 1.0]
        f = (height / 2.0) / math.tan(fov_y / 2.0)
        return cls(tuple(view), f, f, width / 2.0, height / 2.0, width, height, near_plane, far_plane,
                   sh_degree, color_mode)

    def replace(self, **kw) -> "RasterCamera":
        return dataclasses.replace(self, **kw)

    def to_c(self) -> _abi.NpaRasterCamera:
        c = _abi.NpaRasterCamera()
        if len(self.view) != 16:
            raise _abi.InvalidArgument("invalid argument: the view matrix has 16 entries")
        for k, v in enumerate(self.view):
            c.view[k] = float(v)
        c.fx, c.fy, c.cx, c.cy = float(self.fx), float(self.fy), float(self.cx), float(self.cy)
        c.width, c.height = int(self.width), int(self.height)
        c.near_plane, c.far_plane = float(self.near_plane), float(self.far_plane)
        c.sh_degree, c.color_mode = int(self.sh_degree), int(self.color_mode)
        return c


@dataclass
class RolloutConfig:
    """RolloutConfig (crates/burn_automata/src/rollout/mod.rs:102-124)."""

    batch_size: int = 1
    particle_count: int = 4096
    steps: int = 32
    dt: float = 1.0
    update_prob: float = 0.5
    seed: int = 42
    seed_scale: float = 0.2
    extra: dict = field(default_factory=dict)
