"""Device-resident executor: the HIP counterpart of WgpuAutomataExecutor
(crates/burn_automata/src/gpu/types.rs:418-457, crates/burn_automata/src/gpu/executor/*.rs).

A state owns ping-pong particle buffers and every per-step workspace in HBM; a
step is the hashgrid build, the density pass and the fused update, all queued on
the context's stream with no host synchronisation.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import lib
from .config import ALL_VIEWS, GaussianDecodeConfig, HashGridConfig, RenderLossConfig, Splat2dConfig
from .model import NpaModel, NpaWeights
from .runtime import Context, default_context, device_f32, ptr


GAUSSIAN_SH_COEFF_COUNT = 48  # NPA_GAUSSIAN_SH_COEFF_COUNT (gpu_step.wgsl:6)
_EXPORT_KEYS = ("position_visibility", "spherical_harmonic", "rotation", "scale_opacity")


class HipAutomataState:
    def __init__(self, ctx: Context, handle, model: NpaModel, grid: HashGridConfig,
                 batch_size: int, particle_count: int):
        self.ctx = ctx
        self.handle = handle
        self.model = model
        self.grid = grid
        self.batch_size = batch_size
        self.particle_count = particle_count

    @property
    def total(self) -> int:
        return self.batch_size * self.particle_count

    def set_mlp_engine(self, engine: int):
        """The update-MLP engine of this state's steps (_abi.MLP_VALU or _abi.MLP_MFMA)."""
        self.ctx.check(lib().npa_state_set_mlp_engine(self.handle, int(engine)))

    def step_index(self) -> int:
        v = C.c_uint64()
        self.ctx.check(lib().npa_state_step_index(self.handle, C.byref(v)))
        return int(v.value)

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle.value:
            lib().npa_state_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipAutomataExecutor:
    def __init__(self, device: int = 0, ctx: Context | None = None):
        self.ctx = ctx or default_context(device)

    def create_state(self, model: NpaModel, positions, states, batch_size: int,
                     particle_count: int, grid: HashGridConfig, dt: float,
                     update_prob: float = 1.0, seed: int = 0) -> HipAutomataState:
        """create_state_with_update_prob (crates/burn_automata/src/gpu/executor/state.rs:82-111)."""
        model.validate()
        pos = device_f32(positions, device=self.ctx.device).reshape(-1, 4)
        st = device_f32(states, device=self.ctx.device).reshape(-1)
        w = model.weights.to_c()
        h = C.c_void_p()
        self.ctx.check(lib().npa_state_create(
            self.ctx.handle, C.byref(model.config.to_c()), C.byref(w), C.byref(grid.to_c()),
            ptr(pos), ptr(st), batch_size, particle_count, float(dt), float(update_prob),
            int(seed) & 0xFFFFFFFFFFFFFFFF, C.byref(h)))
        return HipAutomataState(self.ctx, h, model, grid, batch_size, particle_count)

    def step_state(self, state: HipAutomataState):
        self.ctx.check(lib().npa_state_step(state.handle, 1))

    def step_state_many(self, state: HipAutomataState, steps: int):
        self.ctx.check(lib().npa_state_step(state.handle, int(steps)))

    def read_state(self, state: HipAutomataState):
        """(positions [n,4], states [n,S], density [n]) as new device tensors."""
        import torch

        dev = f"cuda:{self.ctx.device}"
        pos = torch.empty((state.total, 4), dtype=torch.float32, device=dev)
        st = torch.empty((state.total, state.model.config.state_dims), dtype=torch.float32,
                         device=dev)
        dens = torch.empty(state.total, dtype=torch.float32, device=dev)
        self.ctx.check(lib().npa_state_read(state.handle, ptr(pos), ptr(st), ptr(dens)))
        return pos, st, dens

    def update_state_model(self, state: HipAutomataState, weights):
        w = weights if isinstance(weights, NpaWeights) else NpaWeights.from_arrays(weights,
                                                                                   self.ctx.device)
        w.validate(state.model.config)
        wc = w.to_c()
        self.ctx.check(lib().npa_state_update_model(state.handle, C.byref(wc)))
        state.model = NpaModel(state.model.config, w)

    def splat_2d(self, state: HipAutomataState, cfg: Splat2dConfig):
        import torch

        img = torch.empty((cfg.image_size * cfg.image_size, 4), dtype=torch.float32,
                          device=f"cuda:{self.ctx.device}")
        self.ctx.check(lib().npa_state_splat_2d(state.handle, C.byref(cfg.to_c()), ptr(img)))
        return img

    def splat_2d_tiled(self, state: HipAutomataState, cfg: Splat2dConfig, tiles_x: int):
        """Every system in its own image_size-square window, tiles_x windows per row
        (image [rows * size, tiles_x * size, 4])."""
        import torch

        rows = -(-state.batch_size // tiles_x)
        img = torch.empty((rows * cfg.image_size, tiles_x * cfg.image_size, 4),
                          dtype=torch.float32, device=f"cuda:{self.ctx.device}")
        self.ctx.check(lib().npa_state_splat_2d_tiled(state.handle, C.byref(cfg.to_c()),
                                                      int(tiles_x), ptr(img)))
        return img

    def render_views(self, state: HipAutomataState, cfg: RenderLossConfig, views=ALL_VIEWS):
        """The particle images of mesh_multiview_render_loss_from_trace (render_loss.rs:107-141)
        for the current particles of a batch-1 state: [len(views), size, size, 5]."""
        import torch

        varr = np.ascontiguousarray([int(v) for v in views], dtype=np.uint32)
        img = torch.empty((len(varr), cfg.image_size, cfg.image_size, 5), dtype=torch.float32,
                          device=f"cuda:{self.ctx.device}")
        self.ctx.check(lib().npa_state_render_views(state.handle, varr.ctypes.data_as(C.c_void_p),
                                                    len(varr), C.byref(cfg.to_c()), ptr(img)))
        return img

    def decode_gaussians_3d(self, state: HipAutomataState, cfg: GaussianDecodeConfig):
        import torch

        n = state.total
        K = cfg.sh_coeffs()
        dev = f"cuda:{self.ctx.device}"
        pv = torch.empty((n, 4), dtype=torch.float32, device=dev)
        sh = torch.empty((n, K, 3), dtype=torch.float32, device=dev)
        rot = torch.empty((n, 4), dtype=torch.float32, device=dev)
        so = torch.empty((n, 4), dtype=torch.float32, device=dev)
        self.ctx.check(lib().npa_state_decode_gaussians_3d(state.handle, C.byref(cfg.to_c()),
                                                          ptr(pv), ptr(sh), ptr(rot), ptr(so)))
        return {"position_visibility": pv, "spherical_harmonic": sh, "rotation": rot,
                "scale_opacity": so}

    def _gaussian_buffers(self, count: int):
        import torch

        dev = f"cuda:{self.ctx.device}"
        return {"position_visibility": torch.empty((count, 4), dtype=torch.float32, device=dev),
                "spherical_harmonic": torch.empty((count, GAUSSIAN_SH_COEFF_COUNT), dtype=torch.float32, device=dev),
                "rotation": torch.empty((count, 4), dtype=torch.float32, device=dev),
                "scale_opacity": torch.empty((count, 4), dtype=torch.float32, device=dev)}

    def write_gaussians(self, state: HipAutomataState, buffers=None):
        """write_state_into_gaussian_bind_group (crates/burn_automata/src/gpu/executor/steps.rs:71-108):
        the viewer's planar Gaussian export of the current particles (write_gaussian_from_output,
        gpu_step.wgsl:4963-5052) into `buffers` (new device tensors when None)."""
        g = buffers or self._gaussian_buffers(state.total)
        count = g["position_visibility"].shape[0]
        self.ctx.check(lib().npa_state_write_gaussians(state.handle, count, *(ptr(g[k]) for k in _EXPORT_KEYS)))
        return g

    def step_state_into_gaussians(self, state: HipAutomataState, steps: int = 1, buffers=None):
        """step_state_into_gaussians / step_state_many_into_gaussian_bind_group (steps.rs:111-257):
        max(steps, 1) steps, then the export of the last step's particles. Returns the buffers."""
        g = buffers or self._gaussian_buffers(state.total)
        count = g["position_visibility"].shape[0]
        self.ctx.check(lib().npa_state_step_into_gaussians(state.handle, int(steps), count,
                                                           *(ptr(g[k]) for k in _EXPORT_KEYS)))
        return g

    def raster_gaussians_3d(self, state: HipAutomataState, cfg, camera):
        """The EWA raster (npa_state_raster_gaussians_3d) of the current particles: [height, width, 4].
        cfg None draws the viewer's export (48 SH coefficients at degree 3); a GaussianDecodeConfig
        draws decode_gaussians_3d's colours as RGB. The call sets the camera's colour mode and degree."""
        import torch

        img = torch.empty((camera.height, camera.width, 4), dtype=torch.float32,
                          device=f"cuda:{self.ctx.device}")
        cfg_c = None if cfg is None else C.byref(cfg.to_c())
        self.ctx.check(lib().npa_state_raster_gaussians_3d(state.handle, cfg_c, C.byref(camera.to_c()), ptr(img)))
        return img

    def pair_counts(self, state: HipAutomataState):
        """(candidates visited, pairs accepted) of the neighbour walk on the current particles."""
        c = self.work_counts(state)
        return c["candidates"], c["pairs"]

    def work_counts(self, state: HipAutomataState):
        """Exact work of the state's next step: candidates and pairs of the density pass over every
        particle, and the update mask's targets with their candidates and pairs (the particles the
        second pass and the update MLP process)."""
        v = [C.c_uint64() for _ in range(5)]
        self.ctx.check(lib().npa_state_pair_counts(state.handle, *[C.byref(x) for x in v]))
        keys = ("candidates", "pairs", "targets", "target_candidates", "target_pairs")
        return {k: int(x.value) for k, x in zip(keys, v)}

    def wait_idle(self):
        self.ctx.synchronize()
