"""The compiled learner step of RecurrentPuPO (boonta/algorithms/recurrent_pupo.py:100-308).

``PuPOExecutor`` runs the GRU learner of ``RecurrentExecutor`` with
RecurrentPuPO's minibatching.  One update is this fixed launch sequence on
one stream:

    bootstrap (the tail sequence, as RecurrentPPO)    recurrent_pupo.py:193-203
    ratio [N, T] = 1                                   :306
    keys = split(key, E * M)                           :303-305
    per minibatch step s (:222-301):
        V-trace on the carried ratio: rho = min(ratio, advantage_clip),
        c = min(ratio, trace_clip)                     :210-220, :226
        priorities, probabilities, width = N / M env draws with replacement
        on keys[s], importance weights                 :228-236
        the drawn envs' sample rows (time-major)
        minibatch advantages: normalised over the minibatch, times each
        env's weight, written at the rows' sample indices    :244-250
        the recurrent minibatch of RecurrentPPO from carry[0][envs] (its
        fused loss also writes every row's ratio into ratio[env, t]:
        the scatter of :297), gradient assembly, clip + Adam

An env drawn twice contributes its rows twice, as the gathered trajectory
of the reference does; both copies compute the same values, so the two
writes of its advantages and ratios agree.  The env draws, their weights and
the ratio stay on the device (``IDX``, ``WEIGHTS``, ``RATIO``).
"""
from __future__ import annotations

import torch

from .learner import _p
from .learner_rnn import RecurrentExecutor


class PuPOExecutor(RecurrentExecutor):
    """One compiled RecurrentPuPO.update for fixed (T, N, obs, minibatches, epochs)."""

    beta = 0.2  # importance_exponent(state.step), set by the algorithm before each issue
    # the loss reads each step's own weighted advantages (no per-update records)
    RECORDS = False

    def _alloc_extra(self):
        super()._alloc_extra()
        S, N, T, Bm = self.E * self.M, self.N, self.T, self.Bm
        dev = self.flat.device
        self.KEYS = torch.zeros(S, 2, dtype=torch.int32, device=dev)
        self.IDX = torch.zeros(S, Bm, dtype=torch.int32, device=dev)
        self.WEIGHTS = torch.zeros(S, Bm, dtype=torch.float32, device=dev)
        self.PROB = torch.zeros(N, dtype=torch.float32, device=dev)
        self.RATIO = torch.zeros(N, T, dtype=torch.float32, device=dev)
        # the minibatch's normalised, weighted advantages at their sample indices
        self.ADVW = torch.zeros(self.B, dtype=torch.float32, device=dev)

    def _loss_adv(self) -> int:
        return _p(self.ADVW)

    def _ratio_out(self):
        return _p(self.RATIO), self.N, self.T

    def issue(self, st: int, max_steps: int | None = None):
        inp, cfg = self.inp, self.cfg
        T, N, mb, Bm = self.T, self.N, self.mb, self.Bm
        S = self.E * self.M
        if not self.trunk:
            raise NotImplementedError("the recurrent learner needs an MLP feature extractor before the GRU")
        self._clear_recurrence_error(st)
        self._bootstrap(st)
        self._call("ppo_fill_f32", st, _p(self.RATIO), N * T, 1.0)
        self._call("ppo_threefry_split", st, _p(self.KEY), _p(self.KEYS), S)
        for step in range(S):
            if max_steps is not None and step >= max_steps:
                self._finish_logs(st, step)
                return
            self._call("ppo_vtrace_f32", st, inp["reward"], inp["terminated"], inp["truncated"], inp["value"],
                       _p(self.BOOT), _p(self.RATIO), T, float(cfg.advantage_clip), float(cfg.trace_clip),
                       _p(self.ADV), _p(self.RET), T, N, float(cfg.gamma), float(cfg.gae_lambda), 0)
            envs = _p(self.IDX) + 4 * step * Bm
            weights = _p(self.WEIGHTS) + 4 * step * Bm
            self._call("ppo_priority_choice_f32", st, _p(self.ADV), N, T, N, float(cfg.priority_exponent),
                       float(self.beta), _p(self.KEYS) + 8 * step, Bm, envs, weights, _p(self.PROB))
            rows = _p(self.ROWS) + 4 * step * mb
            self._call("ppo_sequence_rows", st, envs, 1, T, N, Bm, rows)
            self._call("ppo_pupo_advantages_f32", st, _p(self.ADV), rows, mb, weights, Bm,
                       int(cfg.normalize_advantage), _p(self.ADVW))
            self._sequence_minibatch(st, rows, envs, step)
            self._optimizer_step(st, step)
        self._finish_logs(st, S)
        self._call("ppo_count_advance", st, _p(self.flat.count), S, self._abort_word())
