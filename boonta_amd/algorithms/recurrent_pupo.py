"""RecurrentPuPO with the learner update compiled onto MI355X kernels.

Mirrors boonta/algorithms/recurrent_pupo.py:18-308: ``RecurrentPuPOConfig``
(:18-31), ``RecurrentPuPOState`` (:34-38) and ``RecurrentPuPO(cfg, network,
optimizer, importance_exponent=constant_schedule(0.2), auxiliary_losses=(),
advantage_estimator=...)`` with ``init`` (:50-72), ``step`` (:74-98) and
``update(state, key, transitions) -> state`` (:100-308).  ``init`` and
``step`` are RecurrentPPO's (the reference's are the same code); the update
runs on ``PuPOExecutor`` (boonta_amd/learner_pupo.py), captured into one HIP
graph and replayed.  ``transitions`` is laid out as for RecurrentPPO.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable

import numpy as np

from ..learner_pupo import PuPOExecutor
from ..optim import ConstantSchedule, constant_schedule
from .ppo import PPOState
from .recurrent_ppo import RecurrentPPO


@dataclass(frozen=True)
class RecurrentPuPOConfig:
    num_minibatches: int
    update_epochs: int
    clip_coefficient: float
    clip_value_loss: bool
    entropy_coefficient: float
    value_coefficient: float
    gamma: float
    gae_lambda: float
    advantage_clip: float = 1.0
    trace_clip: float = 1.0
    priority_exponent: float = 0.8
    normalize_advantage: bool = True


RecurrentPuPOState = PPOState


@dataclass
class RecurrentPuPO(RecurrentPPO):
    importance_exponent: Callable = field(default_factory=lambda: constant_schedule(0.2))
    executor_class = PuPOExecutor

    def _beta(self, state) -> float:
        """importance_exponent(state.step) (recurrent_pupo.py:208): a constant
        schedule needs no read of the device step counter."""
        sched = self.importance_exponent
        if isinstance(sched, ConstantSchedule):
            return sched.value
        return float(sched(int(state.step.item())))

    def update(self, state, key, transitions):
        T, N = transitions.second.reward.shape[:2]
        obs_dim = int(transitions.first.obs.shape[-1])
        if N % self.cfg.num_minibatches:
            raise ValueError(f"{N} envs are not divisible into {self.cfg.num_minibatches} minibatches")
        ex = self.executor(state, T, N, obs_dim)
        ex.beta = self._beta(state)
        return super().update(state, key, transitions)

    def _graph_key(self, ex) -> tuple:
        # beta is a launch argument of every captured env draw
        return (ex.beta,)

    def logs(self, state, T: int, N: int, obs_dim: int) -> dict:
        """RecurrentPPO's logged scalars plus actor/priority_weight (the mean
        importance weight of each step's draw) and actor/priority_beta
        (recurrent_pupo.py:272-285)."""
        out = super().logs(state, T, N, obs_dim)
        ex = self.executor(state, T, N, obs_dim)
        w = ex.WEIGHTS.detach().cpu().numpy()
        out["actor/priority_weight"] = w.mean(axis=1, dtype=np.float64).astype(np.float32)
        out["actor/priority_beta"] = np.full(len(w), ex.beta, np.float32)
        return out
