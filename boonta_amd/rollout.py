"""The rollout-side ``PPO.step`` on MI355X kernels (boonta/algorithms/ppo.py:57-74).

``StepExecutor`` binds an MLP program to a number of environments and issues,
on one stream:

    network forward on timestep.obs [rows, obs]     network.py:18-49 (shared
        trunk or separate actor / critic towers, as in the learner)
    head GEMMs -> logits or mean, and the value column
    sample_and_log_prob(seed=key)                   distributions.py:8-57
        (``ppo_sample_categorical_f32`` / ``ppo_sample_gaussian_f32``)

``RecurrentStepExecutor`` is the same for ``RecurrentPPO.step``
(recurrent_ppo.py:71-96): trunk forward, the GRU input projection, one GRU
step from the given carry with the carry reset to zeros where the timestep is
done (reset_carry, networks/blocks/rnn.py:11-16,43-46), the heads on the new
carry, and the sampling launch.

The forward reuses the learner's kernels (``ForwardChain``) and reads the
same flat parameter buffer, so a step issued after an update sees the updated
parameters without a copy.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .learner import (A_ROW, B_KN, EPI_BIAS_ACT, LayerBufs, DenseSpec, FlatState, ForwardChain, Program, _act, _p,
                      forward_bufs,
                      split_forward_bufs)


class StepExecutor(ForwardChain):
    """PPO.step for a fixed number of environments (rows).

    A float32 shared-trunk MLP of 256-wide Dense layers with one activation
    and a categorical head of at most 15 logits (the discrete Anakin network)
    steps in one launch, ``ppo_step_mlp_categorical_f32``; ``fused=False``
    issues the layer-by-layer GEMMs and the sampling launch instead."""

    def __init__(self, program: Program, flat: FlatState, rows: int, fused: bool = True):
        if program.gru is not None:
            raise TypeError("a recurrent program steps through RecurrentPPO")
        super().__init__(program, flat)
        lib = _lib.load()
        if program.action_dim > lib.ppo_sample_max_outputs():
            raise NotImplementedError(f"an action dimension above {lib.ppo_sample_max_outputs()} is not compiled")
        dev = flat.device
        self.rows = rows
        self.trunk = [forward_bufs(s, rows, dev) for s in program.trunk]
        self.actor = [forward_bufs(s, rows, dev) for s in program.actor_layers]
        self.critic = [forward_bufs(s, rows, dev) for s in program.critic_layers]
        for group in (self.trunk, self.actor, self.critic):
            if group:
                split_forward_bufs(group[0], rows, dev, self.bf16)
        f32 = dict(dtype=torch.float32, device=dev)
        ha, hc = program.head_a, program.head_c
        if program.shared_head:
            self.HEAD = torch.zeros(rows, ha.w.ld, **f32)
        else:
            self.HA = torch.zeros(rows, ha.w.ld, **f32)
            self.HC = torch.zeros(rows, hc.w.ld, **f32)
        self.KEY = torch.zeros(2, dtype=torch.int32, device=dev)
        self.fused = fused and self._fusable(lib)

    def _fusable(self, lib) -> bool:
        """Whether the one-launch step kernel covers this program."""
        prog = self.prog
        trunk = prog.trunk
        if (self.bf16 or not prog.shared_head or prog.dist["kind"] != "categorical" or not trunk
                or len(trunk) > lib.ppo_step_mlp_max_layers() or trunk[0].dense.fin > lib.ppo_step_mlp_max_obs()):
            return False
        if len({s.act for s in trunk}) != 1 or any(s.ln is not None for s in trunk):
            return False
        if any(s.fout != 256 or s.ld != 256 or (i > 0 and s.dense.fin != 256) for i, s in enumerate(trunk)):
            return False
        h = prog.head_a
        return h.fin == 256 and h.w.ld <= 16 and prog.head_out == prog.dist["num"] and prog.head_out + 1 <= h.w.ld

    def _head(self, st, x, ldx, h: DenseSpec, out: torch.Tensor):
        """Head Dense on the last features (bias added, no activation)."""
        self._gemm(st, A_ROW, B_KN, x, ldx, None, self.flat.view(h.w), h.w.ld, _p(out), h.w.ld, self.rows,
                   h.w.ld, h.fin, 1, 0, EPI_BIAS_ACT, self.flat.view(h.b) if h.b is not None else None, 0, None,
                   None, 0, None, -1)

    def issue(self, st: int, obs: int, ldo: int, temperature: float, action: int, log_prob: int, value: int,
              key: int | None = None):
        """Enqueues one step on stream handle ``st``: obs is a device pointer
        to [rows, ldo] float32; action [rows] int32 (categorical) or [rows, D]
        float32 (Gaussian), log_prob and value [rows] float32; key a device
        pointer to uint32[2] key data (default: this executor's KEY buffer)."""
        key = _p(self.KEY) if key is None else key
        prog = self.prog
        rows = self.rows
        if self.fused:
            h, n = prog.head_a, len(prog.trunk)
            # host arrays of the trunk's kernel / bias pointers (read at launch)
            ws = (ctypes.c_void_p * n)(*[self.flat.view(s.dense.w) for s in prog.trunk])
            lds = (ctypes.c_int64 * n)(*[s.ld for s in prog.trunk])
            bs = (ctypes.c_void_p * n)(*[self.flat.view(s.dense.b) if s.dense.b is not None else None
                                         for s in prog.trunk])
            self._call("ppo_step_mlp_categorical_f32", st, obs, ldo, rows, prog.trunk[0].dense.fin, n, ws, lds, bs, _act(prog.trunk[0].act), self.flat.view(h.w), h.w.ld,
                       self.flat.view(h.b) if h.b is not None else None, prog.dist["num"], key, float(temperature),
                       action, log_prob, value)
            return
        if prog.shared_head:
            x, ldx, _ = self._fwd_layers(st, self.trunk, obs, ldo, None, rows)
            self._head(st, x, ldx, prog.head_a, self.HEAD)
            head, ldh = self.HEAD, self.HEAD.shape[1]
            vsrc, ldv = _p(self.HEAD) + 4 * prog.head_out, ldh
        else:
            xa, lda, _ = self._fwd_layers(st, self.actor, obs, ldo, None, rows)
            self._head(st, xa, lda, prog.head_a, self.HA)
            xc, ldc, _ = self._fwd_layers(st, self.critic, obs, ldo, None, rows)
            self._head(st, xc, ldc, prog.head_c, self.HC)
            head, ldh = self.HA, self.HA.shape[1]
            vsrc, ldv = _p(self.HC), self.HC.shape[1]
        dist = prog.dist
        if dist["kind"] == "categorical":
            self._call("ppo_sample_categorical_f32", st, _p(head), ldh, rows, dist["num"], vsrc, ldv, key,
                       float(temperature), action, log_prob, value)
        else:
            D = dist["dim"]
            if prog.scale_region is not None:
                scale, lds = self.flat.view(prog.scale_region), 0
            else:
                scale, lds = _p(head) + 4 * D, ldh
            self._call("ppo_sample_gaussian_f32", st, _p(head), ldh, scale, lds, rows, D, vsrc, ldv, key,
                       float(temperature), action, D, log_prob, value)

    def record(self, *issue_args) -> list:
        """The launch sequence of one step as (entry point, args) without
        running it (used by the benchmark to time single launches)."""
        calls = []
        self._call = lambda name, *args: calls.append((name, args))
        try:
            self.issue(0, *issue_args)
        finally:
            self._call = _lib.call
        return calls


class RecurrentStepExecutor(ForwardChain):
    """RecurrentPPO.step for a fixed number of environments (rows): the
    network of ``Network(feature_extractor=<MLP>, torso=RNN(GRUCell(H)),
    head=ActorCritic(Dense, Dense))`` one time step at a time."""

    def __init__(self, program: Program, flat: FlatState, rows: int):
        if program.gru is None:
            raise TypeError("RecurrentStepExecutor needs a program with a GRU torso")
        if not program.shared_head or not program.trunk:
            raise NotImplementedError("the recurrent step compiles an MLP feature extractor, the GRU and plain "
                                      "Dense heads")
        if program.dist["kind"] != "categorical":
            raise NotImplementedError("the recurrent step compiles a categorical head")
        super().__init__(program, flat)
        lib = _lib.load()
        if program.action_dim > lib.ppo_sample_max_outputs():
            raise NotImplementedError(f"an action dimension above {lib.ppo_sample_max_outputs()} is not compiled")
        dev = flat.device
        H = program.gru.H
        f32 = dict(dtype=torch.float32, device=dev)
        self.rows = rows
        self.trunk: list[LayerBufs] = [forward_bufs(s, rows, dev) for s in program.trunk]
        self.XI = torch.zeros(rows, 3 * H, **f32)
        self.HEAD = torch.zeros(rows, program.head_a.w.ld, **f32)
        self.KEY = torch.zeros(2, dtype=torch.int32, device=dev)

    def issue(self, st: int, obs: int, ldo: int, carry: int, terminated: int | None, truncated: int | None,
              temperature: float, carry_out: int, action: int, log_prob: int, value: int, key: int | None = None):
        """Enqueues one step: obs [rows, ldo] and carry [rows, H] float32 in,
        terminated / truncated [rows] bool (or None: no reset); the new carry
        [rows, H], action [rows] int32, log_prob and value [rows] out."""
        key = _p(self.KEY) if key is None else key
        prog = self.prog
        g = prog.gru
        H, I = g.H, g.fin
        rows = self.rows
        x, ldx, _ = self._fwd_layers(st, self.trunk, obs, ldo, None, rows)
        self._gemm(st, A_ROW, B_KN, x, ldx, None, self.flat.view(g.wi), 3 * H, _p(self.XI), 3 * H, rows, 3 * H, I,
                   1, 0, EPI_BIAS_ACT, self.flat.view(g.bi), 0, None, None, 0, None, -1)
        self._call("ppo_gru_fwd_step_f32", st, _p(self.XI), 3 * H, carry, H, None, terminated, truncated, None,
                   self.flat.view(g.wh), 3 * H, self.flat.view(g.bhn), carry_out, H, None, H, None, 4 * H, rows, H)
        h = prog.head_a
        self._gemm(st, A_ROW, B_KN, carry_out, H, None, self.flat.view(h.w), h.w.ld, _p(self.HEAD), h.w.ld, rows,
                   h.w.ld, h.fin, 1, 0, EPI_BIAS_ACT, self.flat.view(h.b) if h.b is not None else None, 0, None,
                   None, 0, None, -1)
        ldh = self.HEAD.shape[1]
        self._call("ppo_sample_categorical_f32", st, _p(self.HEAD), ldh, rows, prog.dist["num"],
                   _p(self.HEAD) + 4 * prog.head_out, ldh, key, float(temperature), action, log_prob, value)

    def record(self, *issue_args) -> list:
        calls = []
        self._call = lambda name, *args: calls.append((name, args))
        try:
            self.issue(0, *issue_args)
        finally:
            self._call = _lib.call
        return calls
