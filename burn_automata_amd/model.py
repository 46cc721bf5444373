"""NpaWeights / NpaModel on the HIP path (crates/burn_automata/src/model.rs:12-940)."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import _abi
from ._lib import lib
from .config import HashGridConfig, NpaConfig
from .runtime import default_context, device_f32, ptr


@dataclass
class NpaWeights:
    """Row-major w1[H][F], b1[H], w2[O][H], b2[O] as device tensors."""

    w1: object
    b1: object
    w2: object
    b2: object

    @staticmethod
    def from_arrays(weights, device: int = 0) -> "NpaWeights":
        get = (lambda k: weights[k]) if isinstance(weights, dict) else (lambda k: getattr(weights, k))
        return NpaWeights(*(device_f32(get(k), device=device).reshape(-1)
                            for k in ("w1", "b1", "w2", "b2")))

    def validate(self, config: NpaConfig):
        """NpaWeights::validate (model.rs:76-108)."""
        F, H, O = config.perception_dims(), config.hidden_dims, config.update_dims()
        for name, t, want in (("w1", self.w1, H * F), ("b1", self.b1, H), ("w2", self.w2, O * H),
                              ("b2", self.b2, O)):
            if t.numel() != want:
                raise _abi.InvalidModel(f"{name} len {t.numel()} != {want}")

    def to_c(self) -> _abi.NpaWeightsC:
        return _abi.NpaWeightsC(ptr(self.w1), ptr(self.b1), ptr(self.w2), ptr(self.b2))


@dataclass
class StepOutput:
    """StepOutput (model.rs:737-744): next particles and the perception density."""

    next_positions: object
    next_states: object
    density: object


class NpaModel:
    def __init__(self, config: NpaConfig, weights, device: int = 0):
        self.config = config
        self.weights = weights if isinstance(weights, NpaWeights) else \
            NpaWeights.from_arrays(weights, device)

    def validate(self):
        if self.config.spatial_dims not in (2, 3):
            raise _abi.InvalidModel(
                f"spatial_dims must be 2 or 3, got {self.config.spatial_dims}")
        self.weights.validate(self.config)

    def step(self, positions, states, batch_size: int, particle_count: int,
             grid: HashGridConfig, dt: float, update_mask=None, ctx=None) -> StepOutput:
        """NpaModel::step_cpu (model.rs:768-858) as one fused device step."""
        import torch

        self.validate()
        ctx = ctx or default_context()
        total = batch_size * particle_count
        S = self.config.state_dims
        pos = device_f32(positions, device=ctx.device).reshape(-1, 4)
        st = device_f32(states, device=ctx.device).reshape(-1)
        if pos.shape[0] != total:
            raise _abi.PositionShape(f"positions length {pos.shape[0]} != {total}")
        if st.numel() != total * S:
            raise _abi.StateShape(f"state length {st.numel()} != {total * S}")
        m = None if update_mask is None else device_f32(update_mask, device=ctx.device).reshape(-1)
        op = torch.empty_like(pos)
        os_ = torch.empty_like(st)
        dens = torch.empty(total, dtype=torch.float32, device=pos.device)
        w = self.weights.to_c()
        ctx.check(lib().npa_step(ctx.handle, ptr(pos), ptr(st), batch_size, particle_count,
                                 C.byref(grid.to_c()), C.byref(self.config.to_c()), C.byref(w),
                                 float(dt), ptr(m), ptr(op), ptr(os_), ptr(dens)))
        return StepOutput(op, os_.reshape(total, S), dens)

    def forward_from_features_with_eps(self, features, eps: float, ctx=None):
        """forward_from_features_with_eps (model.rs:867-898): (dx [rows,4], ds [rows,S])."""
        import torch

        ctx = ctx or default_context()
        F = self.config.perception_dims()
        f = device_f32(features, device=ctx.device).reshape(-1, F)
        rows = f.shape[0]
        dx = torch.empty((rows, 4), dtype=torch.float32, device=f.device)
        ds = torch.empty((rows, self.config.state_dims), dtype=torch.float32, device=f.device)
        w = self.weights.to_c()
        ctx.check(lib().npa_mlp_forward(ctx.handle, ptr(f), rows, C.byref(self.config.to_c()),
                                        C.byref(w), float(eps), ptr(dx), ptr(ds)))
        return dx, ds
