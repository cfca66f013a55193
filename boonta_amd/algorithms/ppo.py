"""PPO with the learner update compiled onto MI355X kernels.

Mirrors boonta/algorithms/ppo.py:17-233: ``PPOConfig`` (:17-27), ``PPOState``
(:30-34) and ``PPO(cfg, network, optimizer, auxiliary_losses=(),
advantage_estimator=generalized_advantage_estimator)`` with ``init`` (:45-55),
``step`` (:57-74) and ``update(state, key, transitions) -> state`` (:76-233).

``step`` runs the network forward and the head's sample_and_log_prob as HIP
kernels (see ``rollout.StepExecutor``).

``update`` runs bootstrap, GAE, the epoch permutations and every minibatch
forward/backward/clip/Adam step as HIP kernels (see ``learner.MLPExecutor``);
by default the whole update is captured once into a HIP graph per input
layout and replayed.  Like the reference's jitted update with
``donate_argnames=("state",)`` (podracers/anakin.py:173-179), the state's
buffers are updated in place and the returned state shares them.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable

import numpy as np
import torch

from .. import _lib
from ..flat import load_tree, tree_from_flat
from ..learner import FlatState, MLPExecutor, Program
from ..optim import EmptyState, ScaleByAdamState, as_chain
from ..random import key_data
from ..rollout import StepExecutor
from .advantage_estimators import generalized_advantage_estimator


@dataclass(frozen=True)
class PPOConfig:
    num_minibatches: int
    update_epochs: int
    clip_coefficient: float
    clip_value_loss: bool
    entropy_coefficient: float
    value_coefficient: float
    gamma: float
    gae_lambda: float
    normalize_advantage: bool = False


@dataclass(frozen=True)
class PPOState:
    step: Any
    params: Any
    optimizer_state: Any

    def replace(self, **kw) -> "PPOState":
        import dataclasses
        return dataclasses.replace(self, **kw)


def flat_state_of(state) -> FlatState:
    """The flat device storage behind a state's parameter tree: every leaf is
    a view of the flat parameter buffer, which carries its FlatState (so the
    storage, its compiled updates and their graphs live as long as the state's
    parameters do)."""
    leaf = _first_leaf(state.params)
    base = leaf._base if isinstance(leaf, torch.Tensor) and leaf._base is not None else leaf
    flat = getattr(base, "_flat_state", None)
    if flat is None:
        raise ValueError("this state was not created by PPO.init of this package")
    return flat


def _first_leaf(tree):
    while isinstance(tree, dict):
        tree = tree[sorted(tree)[0]]
    return tree


@dataclass
class PPO:
    cfg: PPOConfig
    network: Any
    optimizer: Any
    auxiliary_losses: tuple = ()
    advantage_estimator: Callable = generalized_advantage_estimator
    use_graph: bool = True
    device: Any = "cuda"

    def __post_init__(self):
        if self.auxiliary_losses:
            raise NotImplementedError("auxiliary losses are not compiled into the learner")
        if self.advantage_estimator is not generalized_advantage_estimator:
            raise NotImplementedError("only the built-in GAE estimator is compiled into the learner")
        self.chain = as_chain(self.optimizer)
        self._programs: dict = {}

    # ------------------------------------------------------------------ init
    def program(self, obs_dim: int) -> Program:
        if obs_dim not in self._programs:
            self._programs[obs_dim] = Program(self.network.plan(obs_dim))
        return self._programs[obs_dim]

    def init(self, key, timestep) -> tuple[PPOState, None]:
        obs_dim = int(timestep.obs.shape[-1])
        prog = self.program(obs_dim)
        flat = FlatState(prog, torch.device(self.device))
        load_tree(prog.layout, flat.P, self.network.init(key_data(key), obs_dim)["params"])
        return self._state(flat), None

    def init_from_params(self, params: dict, obs_dim: int) -> PPOState:
        """A fresh state whose parameters are copied from a nested dict
        (``{"params": {...}}`` of numpy arrays or tensors)."""
        prog = self.program(obs_dim)
        flat = FlatState(prog, torch.device(self.device))
        load_tree(prog.layout, flat.P, params["params"] if "params" in params else params)
        return self._state(flat)

    def _state(self, flat: FlatState) -> PPOState:
        flat.P._flat_state = flat
        lay = flat.program.layout
        opt_state = (EmptyState(), (ScaleByAdamState(count=flat.count[0], mu=tree_from_flat(lay, flat.MU),
                                                     nu=tree_from_flat(lay, flat.NU)), EmptyState()))
        return PPOState(step=torch.zeros((), dtype=torch.int64, device=flat.device),
                        params={"params": tree_from_flat(lay, flat.P)}, optimizer_state=opt_state)

    # ------------------------------------------------------------------ step
    step_class = StepExecutor

    def step_executor(self, state, rows: int, obs_dim: int):
        flat = flat_state_of(state)
        k = (self.step_class, rows, obs_dim)
        if k not in flat.steppers:
            flat.steppers[k] = self.step_class(self.program(obs_dim), flat, rows)
        return flat.steppers[k]

    @staticmethod
    def _set_key(ex, key):
        if isinstance(key, torch.Tensor) and key.is_cuda:
            if key.numel() != 2 or key.element_size() != 4:
                raise ValueError("a device key must hold two 32-bit words")
            ex.KEY.copy_(key.reshape(2).view(torch.int32))
        else:
            ex.KEY.copy_(torch.from_numpy(key_data(key).view(np.int32).copy()))

    def step(self, state, carry, key, timestep, temperature: float = 1.0):
        """Acts on ``timestep.obs`` [N, obs] (ppo.py:57-74): the network forward
        with the current parameters, then ``dist.sample_and_log_prob(seed=key)``.
        Returns (state, carry, action, {"log_prob": [N], "value": [N]}); action
        is int32 [N] (categorical) or float32 [N, D] (Gaussian).  ``key`` is
        key data (host or device) used as given, like the reference's seed."""
        obs = timestep.obs
        if (not isinstance(obs, torch.Tensor) or obs.dtype != torch.float32 or obs.dim() != 2
                or not obs.is_contiguous() or not obs.is_cuda):
            raise TypeError("timestep.obs must be a contiguous float32 [N, obs] device tensor")
        N, obs_dim = (int(d) for d in obs.shape)
        ex = self.step_executor(state, N, obs_dim)
        self._set_key(ex, key)
        dev = ex.KEY.device
        dist = ex.prog.dist
        if dist["kind"] == "categorical":
            action = torch.empty(N, dtype=torch.int32, device=dev)
        else:
            action = torch.empty(N, dist["dim"], dtype=torch.float32, device=dev)
        log_prob = torch.empty(N, dtype=torch.float32, device=dev)
        value = torch.empty(N, dtype=torch.float32, device=dev)
        ex.issue(torch.cuda.current_stream().cuda_stream, obs.data_ptr(), obs_dim, float(temperature),
                 action.data_ptr(), log_prob.data_ptr(), value.data_ptr())
        return state, carry, action, {"log_prob": log_prob, "value": value}

    # ---------------------------------------------------------------- update
    @staticmethod
    def _need(t, dtype, name, shape=None):
        if not isinstance(t, torch.Tensor) or t.dtype != dtype or not t.is_contiguous() or not t.is_cuda:
            raise TypeError(f"{name} must be a contiguous {dtype} device tensor")
        if shape is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
        return t.data_ptr()

    def _inputs(self, transitions, obs_dim: int) -> tuple[dict, tuple]:
        f, s, aux = transitions.first, transitions.second, transitions.aux
        T, N = s.reward.shape[:2]
        need = self._need

        prog = self.program(obs_dim)
        if prog.dist["kind"] == "categorical":
            act = need(s.action, torch.int32, "second.action", (T, N))
        else:
            act = need(s.action, torch.float32, "second.action", (T, N, prog.dist["dim"]))
        sobs = s.obs
        if sobs.dtype != torch.float32 or sobs.shape[-1] != obs_dim or not sobs[-1].is_contiguous():
            raise TypeError("second.obs must be float32 [T, N, obs] with a contiguous last step")
        inp = {
            "obs": need(f.obs, torch.float32, "first.obs", (T, N, obs_dim)),
            "next_obs_last": sobs[-1].data_ptr(),
            "action": act,
            "reward": need(s.reward, torch.float32, "second.reward", (T, N)),
            "terminated": need(s.terminated, torch.bool, "second.terminated", (T, N)),
            "truncated": need(s.truncated, torch.bool, "second.truncated", (T, N)),
            "log_prob": need(aux["log_prob"], torch.float32, "aux['log_prob']", (T, N)),
            "value": need(aux["value"], torch.float32, "aux['value']", (T, N)),
        }
        return inp, tuple(sorted(inp.items()))

    def _stage(self, transitions, own: dict) -> list:
        """(source, destination) pairs that copy a transition into an
        executor's own input buffers."""
        f, s, aux = transitions.first, transitions.second, transitions.aux
        T = s.reward.shape[0]
        return [(f.obs, own["obs"][:T]), (s.obs[-1], own["obs"][T]), (s.action, own["action"]),
                (s.reward, own["reward"]), (s.terminated, own["terminated"]), (s.truncated, own["truncated"]),
                (aux["log_prob"], own["log_prob"]), (aux["value"], own["value"])]

    def _transition_of(self, own: dict):
        """A Transition whose leaves are views of an executor's input buffers."""
        from ..types import Timestep, Transition
        obs = own["obs"]
        return Transition(first=Timestep(obs=obs[:-1]),
                          second=Timestep(obs=obs[1:], action=own["action"], reward=own["reward"],
                                          terminated=own["terminated"], truncated=own["truncated"]),
                          aux={"log_prob": own["log_prob"], "value": own["value"]})

    def rollout_buffers(self, state, T: int, N: int, obs_dim: int, fill_from=None):
        """The input buffers the captured update reads, as a Transition of
        [T, N, ...] device tensors (first.obs and second.obs are views of one
        [T + 1, N, obs] buffer).  A rollout written into them is updated with
        no copy; any other transition is copied into them first.  ``fill_from``
        (a transition of the same shapes) is copied in now."""
        own = self.executor(state, T, N, obs_dim).input_buffers()
        if fill_from is not None:
            self._inputs(fill_from, obs_dim)
            for src, dst in self._stage(fill_from, own):
                dst.copy_(src)
        return self._transition_of(own)

    executor_class = MLPExecutor

    def executor(self, state, T: int, N: int, obs_dim: int) -> MLPExecutor:
        flat = flat_state_of(state)
        k = (self.executor_class, self.cfg, self.chain, T, N, obs_dim)
        if k not in flat.executors:
            flat.executors[k] = self.executor_class(self.program(obs_dim), flat, self.cfg, self.chain, T, N)
        return flat.executors[k]

    # Captured graphs kept per executor (one unless a launch argument such as
    # RecurrentPuPO's importance exponent varies between updates).
    MAX_GRAPHS = 4

    def update(self, state: PPOState, key, transitions) -> PPOState:
        s = transitions.second
        T, N = s.reward.shape[:2]
        obs_dim = int(transitions.first.obs.shape[-1])
        inp, _ = self._inputs(transitions, obs_dim)
        ex = self.executor(state, T, N, obs_dim)
        kd = torch.from_numpy(key_data(key).view(np.int32).copy())
        ex.KEY.copy_(kd, non_blocking=False)
        if not self.use_graph:
            ex.bind(inp)
            ex.issue(torch.cuda.current_stream().cuda_stream)
            return state
        # The graph reads the executor's own input buffers: a transition held
        # elsewhere is copied into them (leaves that already are them are not).
        own = ex.input_buffers()
        for src, dst in self._stage(transitions, own):
            if src.data_ptr() != dst.data_ptr():
                dst.copy_(src)
        ex.bind(self._inputs(self._transition_of(own), obs_dim)[0])
        gk = self._graph_key(ex)
        g = ex.graphs.get(gk)
        if g is None:
            flat = ex.flat
            # An eager pass first loads every kernel; the state is then put back
            # so that the captured graph's replay is this call's one update.
            snapshot = [t.clone() for t in (flat.P, flat.MU, flat.NU, flat.count)]
            ex.issue(torch.cuda.current_stream().cuda_stream)
            for dst, src in zip((flat.P, flat.MU, flat.NU, flat.count), snapshot):
                dst.copy_(src)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                with torch.cuda.graph(g, stream=side):
                    ex.issue(torch.cuda.current_stream().cuda_stream)
            torch.cuda.current_stream().wait_stream(side)
            while len(ex.graphs) >= self.MAX_GRAPHS:
                ex.graphs.pop(next(iter(ex.graphs)))
            ex.graphs[gk] = g
        g.replay()
        return state

    def _graph_key(self, ex) -> tuple:
        """Launch arguments a captured update depends on beyond the executor's
        buffers (none for PPO)."""
        return ()

    def logs(self, state, T: int, N: int, obs_dim: int) -> dict:
        """The logged scalars of every minibatch step of the last update
        (ppo.py:170-179), as numpy arrays of length epochs * minibatches."""
        ex = self.executor(state, T, N, obs_dim)
        L = ex.LOGS.detach().cpu().numpy()
        names = ["actor/loss", "actor/entropy", "actor/approximate_kl", "actor/clip_fraction",
                 "actor/advantage", "critic/loss", "critic/explained_variance", "critic/value", "loss"]
        return {n: L[:, i].copy() for i, n in enumerate(names)}
