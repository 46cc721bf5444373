"""Rollout driver on the device executor.

run_rollout_from_particles (crates/burn_automata/src/rollout/mod.rs:222-297) with the
device update-mask schedule (gpu_step.wgsl:1019-1056): step k of the rollout uses step
index k, the schedule the reference's own GPU-vs-CPU mask test reproduces on the host
(crates/burn_automata/tests/gpu_wgpu/updates.rs:36-86).
"""
from __future__ import annotations

from dataclasses import dataclass

from .config import HashGridConfig, RolloutConfig
from .executor import HipAutomataExecutor
from .model import NpaModel


@dataclass
class RolloutTrace:
    """RolloutTrace (rollout/mod.rs:126-134) without the per-step mean_dx series."""

    positions: object
    states: object
    batch_size: int
    particle_count: int
    state_dims: int
    steps: int


def run_rollout_from_particles(model: NpaModel, grid: HashGridConfig, cfg: RolloutConfig,
                               positions, states, executor: HipAutomataExecutor | None = None
                               ) -> RolloutTrace:
    ex = executor or HipAutomataExecutor()
    state = ex.create_state(model, positions, states, cfg.batch_size, cfg.particle_count, grid,
                            cfg.dt, cfg.update_prob, cfg.seed)
    try:
        ex.step_state_many(state, cfg.steps)
        pos, st, _ = ex.read_state(state)
    finally:
        state.close()
    return RolloutTrace(pos, st, cfg.batch_size, cfg.particle_count, model.config.state_dims,
                        cfg.steps)
