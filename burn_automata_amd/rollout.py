"""Rollout driver on the device executor.

run_rollout_from_particles (crates/burn_automata/src/rollout/mod.rs:222-297) with the
device update-mask schedule (gpu_step.wgsl:1019-1056): step k of the rollout uses step
index k, the schedule the reference's own GPU-vs-CPU mask test reproduces on the host
(crates/burn_automata/tests/gpu_wgpu/updates.rs:36-86).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .config import HashGridConfig, RolloutConfig
from .executor import HipAutomataExecutor
from .kernels import perceive_with_options
from .model import NpaModel


@dataclass
class RolloutTrace:
    """RolloutTrace (rollout/mod.rs:153-161)."""

    positions: object
    states: object
    batch_size: int
    particle_count: int
    state_dims: int
    steps: int
    mean_dx: list = field(default_factory=list)


def mean_dx_norm(dx) -> float:
    """The per-step trace value of rollout/mod.rs:277-282: the Euclidean norm of each particle's
    (x, y, z) motion, squares added left to right, summed over every particle left to right in
    f32 and divided by the particle count (1 for an empty step)."""
    d = np.asarray(dx, dtype=np.float32).reshape(-1, 4)
    if d.shape[0] == 0:
        return 0.0
    norms = np.sqrt(d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1] + d[:, 2] * d[:, 2])
    total = np.add.accumulate(norms, dtype=np.float32)[-1]
    return float(np.float32(total) / np.float32(d.shape[0]))


def run_rollout_from_particles(model: NpaModel, grid: HashGridConfig, cfg: RolloutConfig,
                               positions, states, executor: HipAutomataExecutor | None = None,
                               record_mean_dx: bool = True) -> RolloutTrace:
    """Steps the device state cfg.steps times. With record_mean_dx each step first evaluates the
    update MLP at the current particles for every particle, as step_cpu does before it applies the
    mask (model.rs:768-858), on the device, and records mean_dx_norm of that motion; this adds a
    perception pass, an MLP pass and a device-to-host copy of dx per step."""
    ex = executor or HipAutomataExecutor()
    state = ex.create_state(model, positions, states, cfg.batch_size, cfg.particle_count, grid,
                            cfg.dt, cfg.update_prob, cfg.seed)
    trace_dx = []
    try:
        if record_mean_dx:
            opts = model.config.perception_options()
            for _ in range(cfg.steps):
                pos, st, _ = ex.read_state(state)
                feats = perceive_with_options(pos, st, cfg.batch_size, cfg.particle_count,
                                              model.config.state_dims, grid, opts,
                                              ctx=ex.ctx).features
                dx, _ = model.forward_from_features_with_eps(feats, grid.eps, ctx=ex.ctx)
                trace_dx.append(mean_dx_norm(dx.cpu().numpy()))
                ex.step_state(state)
        else:
            ex.step_state_many(state, cfg.steps)
        pos, st, _ = ex.read_state(state)
    finally:
        state.close()
    return RolloutTrace(pos, st, cfg.batch_size, cfg.particle_count, model.config.state_dims,
                        cfg.steps, trace_dx)
