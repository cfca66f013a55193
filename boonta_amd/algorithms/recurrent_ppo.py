"""RecurrentPPO with the learner update compiled onto MI355X kernels.

Mirrors boonta/algorithms/recurrent_ppo.py:19-281: ``RecurrentPPOConfig``
(:19-28), ``RecurrentPPOState`` (:31-35) and ``RecurrentPPO(cfg, network,
optimizer, auxiliary_losses=(), advantage_estimator=...)`` with ``init``
(:45-69) and ``update(state, key, transitions) -> state`` (:98-281).

``transitions`` is a ``Transition`` of time-major [T, N, ...] device tensors
whose ``first`` timestep carries ``terminated``/``truncated`` (its ``done`` is
the reset flag of each step, recurrent_ppo.py:107-116), and whose ``carry`` is
the [T, N, H] carry sequence the rollout recorded (only ``carry[0]`` and
``carry[-1]`` are read: ``Transition.start`` and ``Transition.tail``,
boonta/utils/transition.py:16-26).  The update runs on ``RecurrentExecutor``
(boonta_amd/learner_rnn.py), captured into one HIP graph and replayed.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ..learner_rnn import RecurrentExecutor
from ..random import key_data
from .ppo import PPO, PPOConfig, PPOState


@dataclass(frozen=True)
class RecurrentPPOConfig(PPOConfig):
    pass


RecurrentPPOState = PPOState


@dataclass
class RecurrentPPO(PPO):
    executor_class = RecurrentExecutor

    def init(self, key, timestep) -> tuple[PPOState, torch.Tensor]:
        """(state, carry): the zero initial carry [N, H] of the GRU
        (rnn.py:56-59), as RecurrentPPO.init returns it (:45-69)."""
        state, _ = super().init(key, timestep)
        plan = self.program(int(timestep.obs.shape[-1])).plan
        n = int(timestep.obs.shape[0])
        carry = torch.zeros(n, plan["torso"]["features"], dtype=torch.float32, device=torch.device(self.device))
        return state, carry

    def _inputs(self, transitions, obs_dim: int) -> tuple[dict, tuple]:
        inp, _ = super()._inputs(transitions, obs_dim)
        f, s = transitions.first, transitions.second
        T, N = s.reward.shape[:2]
        need = self._need
        prog = self.program(obs_dim)
        if prog.gru is None:
            raise TypeError("RecurrentPPO needs a network with an RNN(GRUCell) torso")
        H = prog.gru.H
        carry = transitions.carry
        if carry is None:
            raise ValueError("transitions.carry must hold the rollout's [T, N, H] carry sequence")
        need(carry, torch.float32, "transitions.carry", (T, N, H))
        inp.update({
            "first_terminated": need(f.terminated, torch.bool, "first.terminated", (T, N)),
            "first_truncated": need(f.truncated, torch.bool, "first.truncated", (T, N)),
            "carry0": carry[0].data_ptr(),
            "carry_last": carry[-1].data_ptr(),
        })
        return inp, tuple(sorted(inp.items()))
