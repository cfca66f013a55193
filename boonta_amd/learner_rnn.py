"""The compiled learner step of RecurrentPPO (boonta/algorithms/recurrent_ppo.py:98-281).

``RecurrentExecutor`` extends the MLP executor with the GRU torso of
``Network(feature_extractor=<MLP>, torso=RNN(GRUCell(H)), head=ActorCritic(Dense, Dense))``.
One update is this fixed launch sequence on one stream:

    bootstrap (Transition.tail, transition.py:20-26; recurrent_ppo.py:188-198):
        trunk on first.obs[-1] and second.obs[-1], input projections, two GRU
        steps from carry[-1] with the resets first.done[-1] / second.done[-1],
        value head
    GAE                                              recurrent_ppo.py:199-205
    E permutations of the N envs                     recurrent_ppo.py:269-279
    sample rows of every sequence minibatch          (t * N + env, time-major)
    per minibatch of B = N / M envs x T steps (recurrent_ppo.py:214-267):
        trunk forward (rows gathered in the first GEMM), input projections of
        all T * B rows in one GEMM, T GRU forward steps from carry[0][envs]
        with the resets first.done, fused heads + loss + head backward, T GRU
        backward steps, dWh / dWi / dX GEMMs, trunk backward, gradient
        assembly, clip + Adam

The minibatch keeps its rows time-major (row = t * B + b), so step t of the
recurrence reads and writes one contiguous block; the loss is a mean over all
rows, so the row order does not change it.
"""
from __future__ import annotations

import torch

from . import _lib
from .learner import A_COL, A_ROW, B_KN, B_NK, EPI_BIAS_ACT, EPI_STORE, FlatState, MLPExecutor, Program, _p, _splits


class RecurrentExecutor(MLPExecutor):
    """One compiled RecurrentPPO.update for fixed (T, N, obs, minibatches, epochs)."""

    def __init__(self, program: Program, flat: FlatState, cfg, chain, T: int, N: int):
        if program.gru is None:
            raise TypeError("RecurrentExecutor needs a program with a GRU torso")
        if not program.shared_head:
            raise NotImplementedError("the recurrent learner compiles plain Dense actor and critic heads")
        super().__init__(program, flat, cfg, chain, T, N)
        if not self.fused:
            raise NotImplementedError("the recurrent learner needs the fused head + loss kernel "
                                      "(head width <= 512, at most 15 actions)")

    def _perm_size(self) -> int:
        """RecurrentPPO permutes envs, not samples (recurrent_ppo.py:272)."""
        return self.N

    def _boot_rows(self) -> int:
        """The tail sequence has two steps per env (transition.py:20-26)."""
        return 2 * self.N

    def _alloc_extra(self):
        g = self.prog.gru
        H, I = g.H, g.fin
        dev = self.flat.device
        f32 = dict(dtype=torch.float32, device=dev)
        rows = self.mb
        self.Bm = self.N // self.M
        self.ROWS = torch.zeros(self.E * self.M, rows, dtype=torch.int32, device=dev)
        self.XI = torch.zeros(rows, 3 * H, **f32)
        self.HOUT = torch.zeros(rows, H, **f32)
        self.HP = torch.zeros(rows, H, **f32)
        self.GATES = torch.zeros(rows, 4 * H, **f32)
        self.DHOUT = torch.zeros(rows, H, **f32)
        self.DHS = torch.zeros(rows, H, **f32)
        self.DGATE = torch.zeros(rows, 4 * H, **f32)
        # the recurrence of a minibatch in one launch per direction when all
        # its workgroups fit the device at once (else one launch per step);
        # where they take the shape, the forward launch also makes the input
        # projections (else one GEMM before it) and the backward launch the
        # GRU's weight gradients, one partial per block of 16 sequences (else
        # two GEMMs after it)
        self.seq = self.SEQ and self._seq_fits(self.Bm, H)
        self.seq_dw = self.seq and self.SEQ_DW and H == 256 and I == 256
        self.seq_xw = self.seq and self.SEQ_XW and H == 256 and I == 256
        if self.seq_dw:
            self.wh_splits = self.wi_splits = _lib.load().ppo_gru_seq_dw_parts(self.Bm)
        else:
            self.wh_splits = _splits(rows, H, 3 * H)
            self.wi_splits = _splits(rows, I, 3 * H)
        self.WHPART = torch.zeros(self.wh_splits, H, 3 * H, **f32)
        self.WHBPART = torch.zeros(self.wh_splits, 3 * H, **f32)
        self.WIPART = torch.zeros(self.wi_splits, I, 3 * H, **f32)
        self.WIBPART = torch.zeros(self.wi_splits, 3 * H, **f32)
        n2 = 2 * self.N
        self.XIB = torch.zeros(n2, 3 * H, **f32)
        self.HB = torch.zeros(n2, H, **f32)
        if self.seq:
            lib = _lib.load()
            self.SEQX = torch.zeros(max(1, lib.ppo_gru_seq_exchange_bytes(self.Bm, H) // 8), dtype=torch.int64,
                                    device=dev)
            self.SEQERR = torch.zeros(1, dtype=torch.int32, device=dev)
            # with both fused sequence launches, one ring per direction: each
            # launch leaves the other's ring zero as it finishes, so no zeroing
            # launch runs before either (both zeroed at the start of an update)
            self.SEQX_F = (torch.zeros(max(1, 2 * self.Bm * H), dtype=torch.int64, device=dev)
                           if self.RING_PAIR and self.seq_xw and self.seq_dw else None)

    SEQ = True               # sequence launches where they fit
    SEQ_DW = True            # the weight gradients inside the backward sequence launch where it takes them
    SEQ_XW = True            # the input projections inside the forward sequence launch where it takes them
    SEQ_SPIN = 1 << 18       # polls of a step wait before it gives up (about a second)
    RING_PAIR = True         # one exchange ring per direction, each left zero by the other's launch

    @staticmethod
    def _seq_fits(Bm: int, H: int) -> bool:
        """Whether the one-launch recurrence takes this minibatch: H a multiple
        of 64 up to 256 and every workgroup resident at once."""
        if H % 64 or H > 256 or Bm <= 0:
            return False
        return (Bm + 15) // 16 * (H // 16) <= _lib.load().ppo_gru_seq_max_workgroups()

    def recurrence_error(self) -> bool:
        """True when a wait of a one-launch recurrence of the last update gave
        up; reading it synchronizes.  From that launch on, the update's
        optimizer steps and its count advance wrote nothing (their abort word
        is this error word), so the parameters are those of the last step
        before it."""
        return bool(self.seq and int(self.SEQERR.item()) != 0)

    def _abort_word(self):
        return _p(self.SEQERR) if self.seq else None

    def _ring(self, fwd: bool):
        """(exchange ring) of a fused sequence launch: the forward's own ring
        when the directions have one each, else the shared one."""
        return (_p(self.SEQX_F) if fwd and self.SEQX_F is not None else _p(self.SEQX),)

    def _ring_clear(self, fwd: bool):
        """(ring_is_zero, ring to clear, its bytes) of a fused sequence
        launch: with a ring per direction, its own ring is zero on entry and it
        zeroes the other direction's as it finishes."""
        if self.SEQX_F is None:
            return (0, None, 0)
        other = self.SEQX if fwd else self.SEQX_F
        return (1, _p(other), 8 * other.numel())

    def _clear_recurrence_error(self, st):
        """Zeroes the error word at the start of an update, with a kernel (a
        memset node in a replayed graph is avoided on purpose)."""
        if self.seq:
            self._call("ppo_fill_f32", st, _p(self.SEQERR), 1, 0.0)
            if self.SEQX_F is not None:
                # (also after an update whose recurrence gave up, which may leave a ring unzeroed)
                self._call("ppo_fill_f32", st, _p(self.SEQX), 2 * self.SEQX.numel(), 0.0)
                self._call("ppo_fill_f32", st, _p(self.SEQX_F), 2 * self.SEQX_F.numel(), 0.0)

    def _extra_input_buffers(self) -> dict:
        """first.terminated / first.truncated [T, N] and the carry sequence
        [T, N, H] (only carry[0] and carry[-1] are read)."""
        T, N, dev = self.T, self.N, self.flat.device
        return {"first_terminated": torch.zeros(T, N, dtype=torch.bool, device=dev),
                "first_truncated": torch.zeros(T, N, dtype=torch.bool, device=dev),
                "carry": torch.zeros(T, N, self.prog.gru.H, dtype=torch.float32, device=dev)}

    def _extra_segments(self, G: int) -> list:
        g = self.prog.gru
        H, I = g.H, g.fin
        return [
            (G + 4 * g.wi.offset, _p(self.WIPART), I * 3 * H, I * 3 * H, self.wi_splits, 0),
            (G + 4 * g.bi.offset, _p(self.WIBPART), 3 * H, 3 * H, self.wi_splits, 0),
            (G + 4 * g.wh.offset, _p(self.WHPART), H * 3 * H, H * 3 * H, self.wh_splits, 0),
            # hn's bias gradient is the column sum of dhn, the last H columns
            (G + 4 * g.bhn.offset, _p(self.WHBPART) + 4 * 2 * H, H, 3 * H, self.wh_splits, 0),
        ]

    def _head_a_io(self, la):
        """The heads read the GRU output directly (no activation between)."""
        H = self.prog.gru.H
        return _p(self.HOUT), H, _p(self.DHOUT), 0, None, 0

    # ------------------------------------------------------------------ pieces
    def _trunk_out(self):
        """(pointer, ld) of the trunk's output rows (the GRU input)."""
        if self.trunk:
            lb = self.trunk[-1]
            return _p(lb.Y), lb.spec.ld
        return None, 0

    def _gru_fwd(self, st, xi, hprev, hprev_rows, term, trunc, flag_rows, h_out, hp_out, gates, B):
        g = self.prog.gru
        H = g.H
        self._call("ppo_gru_fwd_step_f32", st, xi, 3 * H, hprev, H, hprev_rows, term, trunc, flag_rows,
                   self.flat.view(g.wh), 3 * H, self.flat.view(g.bhn), h_out, H, hp_out, H, gates, 4 * H, B, H)

    def issue(self, st: int, max_steps: int | None = None):
        inp, cfg = self.inp, self.cfg
        T, N, mb, Bm = self.T, self.N, self.mb, self.Bm
        if not self.trunk:
            raise NotImplementedError("the recurrent learner needs an MLP feature extractor before the GRU")
        self._clear_recurrence_error(st)
        # 1. bootstrap: the two-step tail sequence from carry[-1]
        self._bootstrap(st)
        # 2. GAE
        self._call("ppo_gae_f32", st, inp["reward"], inp["terminated"], inp["truncated"], inp["value"],
                   _p(self.BOOT), None, None, _p(self.ADV), _p(self.RET), T, N, float(cfg.gamma),
                   float(cfg.gae_lambda), 0)
        self._normalize(st)
        self._pack_samples(st)
        # 3. env permutations, and the sample rows of every minibatch
        self._call("ppo_epoch_permutations", st, _p(self.KEY), self.E, N, _p(self.PERM), _p(self.PERM_WS),
                   self.PERM_WS.numel())
        self._call("ppo_sequence_rows", st, _p(self.PERM), self.E * self.M, T, N, Bm, _p(self.ROWS))
        # 4. minibatch steps
        for e in range(self.E):
            for m in range(self.M):
                step = e * self.M + m
                if max_steps is not None and step >= max_steps:
                    self._finish_logs(st, step)
                    return
                rows = _p(self.ROWS) + 4 * step * mb
                envs = _p(self.PERM) + 4 * (e * N + m * Bm)
                self._sequence_minibatch(st, rows, envs, step)
                self._optimizer_step(st, step)
        self._finish_logs(st, self.E * self.M)
        self._call("ppo_count_advance", st, _p(self.flat.count), self.E * self.M, self._abort_word())

    def _bootstrap(self, st):
        """Value of second.obs[-1]: the two-step tail sequence (first[-1],
        second[-1]) from carry[-1] with the resets first.done[-1] /
        second.done[-1] (transition.py:20-26, recurrent_ppo.py:188-198)."""
        inp, prog = self.inp, self.prog
        g = prog.gru
        H, I = g.H, g.fin
        T, N = self.T, self.N
        ldo = self.obs_dim
        last = 4 * (T - 1) * N
        self._fwd_layers(st, self.boot_layers, inp["obs"] + last * ldo, ldo, None, N, row0=0)
        self._fwd_layers(st, self.boot_layers, inp["next_obs_last"], ldo, None, N, row0=N)
        eb = self.boot_layers[-1]
        self._gemm(st, A_ROW, B_KN, _p(eb.Y), eb.spec.ld, None, self.flat.view(g.wi), 3 * H,
                   _p(self.XIB), 3 * H, 2 * N, 3 * H, I, 1, 0, EPI_BIAS_ACT, self.flat.view(g.bi), 0, None, None, 0,
                   None, -1)
        self._gru_fwd(st, _p(self.XIB), inp["carry_last"], None, inp["first_terminated"] + (T - 1) * N,
                      inp["first_truncated"] + (T - 1) * N, None, _p(self.HB), None, None, N)
        self._gru_fwd(st, _p(self.XIB) + 4 * N * 3 * H, _p(self.HB), None, inp["terminated"] + (T - 1) * N,
                      inp["truncated"] + (T - 1) * N, None, _p(self.HB) + 4 * N * H, None, None, N)
        h = prog.head_a
        self._gemm(st, A_ROW, B_KN, _p(self.HB) + 4 * N * H, H, None, self.flat.view(h.w), h.w.ld,
                   _p(self.HEADB), h.w.ld, N, h.w.ld, h.fin, 1, 0, EPI_BIAS_ACT, self.flat.view(h.b), 0, None, None,
                   0, None, -1)
        self._call("ppo_act_fwd_f32", st, _p(self.HEADB) + 4 * prog.head_out, self.HEADB.shape[1], _p(self.BOOT),
                   1, N, 1, 0)

    def _sequence_minibatch(self, st, rows, envs, step):
        inp, prog, cfg = self.inp, self.prog, self.cfg
        g = prog.gru
        H, I = g.H, g.fin
        T, mb, Bm = self.T, self.mb, self.Bm
        ldo = self.obs_dim
        fterm, ftrunc = inp["first_terminated"], inp["first_truncated"]
        # forward: trunk on the gathered rows, input projections of every step
        self._fwd_layers(st, self.trunk, inp["obs"], ldo, rows, mb)
        e_ptr, lde = self._trunk_out()
        if not self.seq_xw:
            self._gemm(st, A_ROW, B_KN, e_ptr, lde, None, self.flat.view(g.wi), 3 * H, _p(self.XI),
                       3 * H, mb, 3 * H, I, 1, 0, EPI_BIAS_ACT, self.flat.view(g.bi), 0, None, None, 0, None, -1)
        blk = Bm * H
        if self.seq_xw:
            self._call("ppo_gru_fwd_seq_xw_f32", st, inp["carry0"], H, envs, fterm, ftrunc, rows, Bm,
                       self.flat.view(g.wh), 3 * H, self.flat.view(g.bhn), _p(self.HOUT), H, blk, _p(self.HP), H,
                       blk, _p(self.GATES), 4 * H, Bm * 4 * H, Bm, H, T, *self._ring(fwd=True), _p(self.SEQERR),
                       self.SEQ_SPIN, e_ptr, lde, Bm * lde, I, self.flat.view(g.wi), 3 * H, self.flat.view(g.bi),
                       *self._ring_clear(fwd=True))
        elif self.seq:
            self._call("ppo_gru_fwd_seq_f32", st, _p(self.XI), 3 * H, Bm * 3 * H, inp["carry0"], H, envs, fterm,
                       ftrunc, rows, Bm, self.flat.view(g.wh), 3 * H, self.flat.view(g.bhn), _p(self.HOUT), H, blk,
                       _p(self.HP), H, blk, _p(self.GATES), 4 * H, Bm * 4 * H, Bm, H, T, _p(self.SEQX),
                       _p(self.SEQERR), self.SEQ_SPIN)
        for t in range(T if not self.seq else 0):
            if t == 0:
                hprev, hrows = inp["carry0"], envs
            else:
                hprev, hrows = _p(self.HOUT) + 4 * (t - 1) * blk, None
            self._gru_fwd(st, _p(self.XI) + 4 * t * Bm * 3 * H, hprev, hrows, fterm, ftrunc, rows + 4 * t * Bm,
                          _p(self.HOUT) + 4 * t * blk, _p(self.HP) + 4 * t * blk,
                          _p(self.GATES) + 4 * t * Bm * 4 * H, Bm)
        # loss and the cotangent of every GRU output
        dist = _lib.DIST[prog.dist["kind"]]
        self._fused_head_loss(st, rows, step, dist, prog.action_dim, None, inp["action"], None)
        # backward through time
        wh = self.flat.view(g.wh)
        G4 = 4 * H
        if self.seq_dw:
            self._call("ppo_gru_bwd_seq_dw_f32", st, wh, 3 * H, fterm, ftrunc, rows, Bm, _p(self.DHOUT), H, blk,
                       _p(self.GATES), G4, Bm * G4, _p(self.HP), H, blk, _p(self.DHS), H, blk, _p(self.DGATE), G4,
                       Bm * G4, Bm, H, T, *self._ring(fwd=False), _p(self.SEQERR), self.SEQ_SPIN, e_ptr, lde,
                       Bm * lde, I, _p(self.WHPART), _p(self.WHBPART), _p(self.WIPART), _p(self.WIBPART),
                       *self._ring_clear(fwd=False))
        elif self.seq:
            self._call("ppo_gru_bwd_seq_f32", st, wh, 3 * H, fterm, ftrunc, rows, Bm, _p(self.DHOUT), H, blk,
                       _p(self.GATES), G4, Bm * G4, _p(self.HP), H, blk, _p(self.DHS), H, blk, _p(self.DGATE), G4,
                       Bm * G4, Bm, H, T, _p(self.SEQX), _p(self.SEQERR), self.SEQ_SPIN)
        else:
            s = T - 1
            self._call("ppo_gru_bwd_step_f32", st, None, 0, None, 0, None, 0, None, 0, None, None, None,
                       _p(self.DHOUT) + 4 * s * blk, H, _p(self.GATES) + 4 * s * Bm * G4, G4,
                       _p(self.HP) + 4 * s * blk, H, _p(self.DHS) + 4 * s * blk, H,
                       _p(self.DGATE) + 4 * s * Bm * G4, G4, Bm, H)
        for t in range(T - 1, 0, -1) if not self.seq else ():
            s = t - 1
            self._call("ppo_gru_bwd_step_f32", st, _p(self.DGATE) + 4 * (t * Bm * G4 + H), G4, wh, 3 * H,
                       _p(self.DHS) + 4 * t * blk, H, _p(self.GATES) + 4 * (t * Bm * G4 + 2 * H), G4, fterm, ftrunc,
                       rows + 4 * t * Bm, _p(self.DHOUT) + 4 * s * blk, H, _p(self.GATES) + 4 * s * Bm * G4, G4,
                       _p(self.HP) + 4 * s * blk, H, _p(self.DHS) + 4 * s * blk, H,
                       _p(self.DGATE) + 4 * s * Bm * G4, G4, Bm, H)
        # recurrent and input kernels: dWh = HP^T [dar|daz|dhn], dWi = E^T [dan|dar|daz]
        if not self.seq_dw:
            self._gemm(st, A_COL, B_KN, _p(self.HP), H, None, _p(self.DGATE) + 4 * H, G4,
                       _p(self.WHPART), 3 * H, H, 3 * H, mb, self.wh_splits, H * 3 * H, EPI_STORE, None, 0, None, None,
                       0, _p(self.WHBPART), -1)
            self._gemm(st, A_COL, B_KN, e_ptr, lde, None, _p(self.DGATE), G4, _p(self.WIPART), 3 * H,
                       I, 3 * H, mb, self.wi_splits, I * 3 * H, EPI_STORE, None, 0, None, None, 0, _p(self.WIBPART),
                       -1)
        # cotangent of the trunk output: [dan|dar|daz] Wi^T, times the trunk's activation derivative
        dst, epi, act, aux, ldaux = self._dx_target(self.trunk[-1])
        self._gemm(st, A_ROW, B_NK, _p(self.DGATE), G4, None, self.flat.view(g.wi), 3 * H, dst,
                   self.trunk[-1].spec.ld, mb, I, 3 * H, 1, 0, epi, None, act, None, aux, ldaux, None, -1)
        self._bwd_layers(st, self.trunk, inp["obs"], ldo, rows)
