"""RecurrentPPO with the learner update compiled onto MI355X kernels.

Mirrors boonta/algorithms/recurrent_ppo.py:19-281: ``RecurrentPPOConfig``
(:19-28), ``RecurrentPPOState`` (:31-35) and ``RecurrentPPO(cfg, network,
optimizer, auxiliary_losses=(), advantage_estimator=...)`` with ``init``
(:45-69), ``step`` (:71-96) and ``update(state, key, transitions) -> state``
(:98-281).  ``step`` runs on ``RecurrentStepExecutor`` (boonta_amd/rollout.py).

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
from ..rollout import RecurrentStepExecutor
from .ppo import PPO, PPOConfig, PPOState


@dataclass(frozen=True)
class RecurrentPPOConfig(PPOConfig):
    pass


class RecurrenceError(RuntimeError):
    """A one-launch GRU recurrence of an update gave up waiting (its bounded
    step wait ran out, e.g. because other work held the GPU's compute units).
    The update's optimizer steps from that point on wrote nothing, so the
    parameters are those of the last optimizer step before it."""


RecurrentPPOState = PPOState


@dataclass
class RecurrentPPO(PPO):
    executor_class = RecurrentExecutor
    step_class = RecurrentStepExecutor

    def init(self, key, timestep) -> tuple[PPOState, torch.Tensor]:
        """(state, carry): the zero initial carry [N, H] of the GRU
        (rnn.py:56-59), as RecurrentPPO.init returns it (:45-69)."""
        state, _ = super().init(key, timestep)
        plan = self.program(int(timestep.obs.shape[-1])).plan
        n = int(timestep.obs.shape[0])
        carry = torch.zeros(n, plan["torso"]["features"], dtype=torch.float32, device=torch.device(self.device))
        return state, carry

    def step(self, state, carry, key, timestep, temperature: float = 1.0):
        """One time step for N envs (recurrent_ppo.py:71-96): the carry is reset
        to zeros where ``timestep`` is done (terminated | truncated; None flags
        reset nothing), the GRU advances one step and the head's action is
        sampled.  Returns (state, new carry [N, H], action int32 [N],
        {"log_prob": [N], "value": [N]}); ``carry`` None is the zero carry."""
        obs = timestep.obs
        if (not isinstance(obs, torch.Tensor) or obs.dtype != torch.float32 or obs.dim() != 2
                or not obs.is_contiguous() or not obs.is_cuda):
            raise TypeError("timestep.obs must be a contiguous float32 [N, obs] device tensor")
        N, obs_dim = (int(d) for d in obs.shape)
        ex = self.step_executor(state, N, obs_dim)
        H = ex.prog.gru.H
        dev = ex.KEY.device
        if carry is None:
            carry = torch.zeros(N, H, dtype=torch.float32, device=dev)
        self._need(carry, torch.float32, "carry", (N, H))
        flags = []
        for name in ("terminated", "truncated"):
            f = getattr(timestep, name)
            flags.append(None if f is None else self._need(f, torch.bool, f"timestep.{name}", (N,)))
        self._set_key(ex, key)
        new_carry = torch.empty(N, H, dtype=torch.float32, device=dev)
        action = torch.empty(N, dtype=torch.int32, device=dev)
        log_prob = torch.empty(N, dtype=torch.float32, device=dev)
        value = torch.empty(N, dtype=torch.float32, device=dev)
        ex.issue(torch.cuda.current_stream().cuda_stream, obs.data_ptr(), obs_dim, carry.data_ptr(), flags[0],
                 flags[1], float(temperature), new_carry.data_ptr(), action.data_ptr(), log_prob.data_ptr(),
                 value.data_ptr())
        return state, new_carry, action, {"log_prob": log_prob, "value": value}

    def update(self, state, key, transitions):
        """RecurrentPPO.update (recurrent_ppo.py:98-281).  Raises
        RecurrenceError when an earlier update's recurrence is known to have
        given up (checked without waiting; ``logs`` waits and checks)."""
        T, N = transitions.second.reward.shape[:2]
        ex = self.executor(state, T, N, int(transitions.first.obs.shape[-1]))
        self._check_recurrence(ex, wait=False)
        state = super().update(state, key, transitions)
        if ex.seq:
            # a copy of the error word that a later call reads once it has landed
            if getattr(ex, "err_host", None) is None:
                ex.err_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
                ex.err_event = torch.cuda.Event()
            ex.err_host.copy_(ex.SEQERR, non_blocking=True)
            ex.err_event.record()
            ex.err_pending = True
        return state

    @staticmethod
    def _check_recurrence(ex, wait: bool):
        if not getattr(ex, "err_pending", False):
            return
        if not wait and not ex.err_event.query():
            return
        ex.err_event.synchronize()
        ex.err_pending = False
        if int(ex.err_host[0]) != 0:
            raise RecurrenceError("a GRU sequence launch gave up waiting for a step of its recurrence: the "
                                  "update stopped applying optimizer steps at that point")

    def logs(self, state, T: int, N: int, obs_dim: int) -> dict:
        """The logged scalars of the last update; raises RecurrenceError when
        its recurrence gave up (its logs then describe no valid update)."""
        ex = self.executor(state, T, N, obs_dim)
        self._check_recurrence(ex, wait=True)
        if ex.recurrence_error():
            raise RecurrenceError("a GRU sequence launch of the last update gave up waiting for a step of its "
                                  "recurrence: the update stopped applying optimizer steps at that point")
        return super().logs(state, T, N, obs_dim)

    def _stage(self, transitions, own: dict) -> list:
        f, carry = transitions.first, transitions.carry
        return super()._stage(transitions, own) + [
            (f.terminated, own["first_terminated"]), (f.truncated, own["first_truncated"]),
            (carry[0], own["carry"][0]), (carry[-1], own["carry"][-1])]

    def _transition_of(self, own: dict):
        tr = super()._transition_of(own)
        first = tr.first.replace(terminated=own["first_terminated"], truncated=own["first_truncated"])
        return tr.replace(first=first, carry=own["carry"])

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
