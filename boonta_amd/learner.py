"""The compiled PPO learner step for MLP actor-critics.

``Program`` lowers a network plan into the flat parameter layout and a tower
structure (trunk layers; actor / critic layers; heads).  ``MLPExecutor``
binds a program to one rollout shape (T, N, minibatches, epochs), owns every
device buffer the update needs, and issues the update as a fixed sequence of
C-ABI launches on one stream:

    bootstrap value  (critic path on second.obs[-1])   ppo.py:208-212
    GAE reverse scan                                    ppo.py:213-219
    E epoch permutations (threefry + radix sort)        ppo.py:199-201,230-231
    per minibatch (ppo.py:148-197):
        forward GEMMs (minibatch rows gathered inside the first GEMM)
        head GEMM -> fused loss + cotangents -> 8 logged scalars
        backward GEMMs (dX with the activation derivative fused, dW split
        over rows with the bias gradient), LayerNorm backward
        gradient assembly (+ global-norm partials), clip + Adam

Because every pointer is fixed once the executor exists, the whole update can
be captured into one HIP graph and replayed (the optax step count and the
PRNG key are read from device memory).
"""
from __future__ import annotations

import ctypes
import math
import struct
import weakref
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .flat import FlatLayout, Region, round_up

EPI_STORE, EPI_BIAS_ACT, EPI_DACT = 0, 1, 2
A_ROW, A_COL = 0, 1          # a_layout: [m][k] / [k][m]
B_KN, B_NK = 0, 1            # b_layout: [k][n] / [n][k]


def _p(t):
    return None if t is None else t.data_ptr()


def _destroy_events(destroy, events):
    for ev in events:
        destroy(ev)


def _act(name):
    return _lib.ACT[name]


# ------------------------------------------------------------------- program
@dataclass
class DenseSpec:
    path: tuple
    fin: int
    fout: int
    w: Region
    b: Region | None


@dataclass
class LayerSpec:
    dense: DenseSpec
    ln: dict | None = None        # {"path", "eps", "scale": Region, "bias": Region}
    act: str | None = None

    @property
    def fout(self):
        return self.dense.fout

    @property
    def ld(self):
        return self.dense.w.ld


def _group(stages):
    """dense [layernorm] [act] groups; returns (layers, trailing dense or None)."""
    layers, i = [], 0
    while i < len(stages):
        st = stages[i]
        if st["op"] != "dense":
            raise NotImplementedError(f"stage {st['op']} must follow a Dense layer")
        layer = {"dense": st, "ln": None, "act": None}
        i += 1
        if i < len(stages) and stages[i]["op"] == "layernorm":
            layer["ln"] = stages[i]
            i += 1
        if i < len(stages) and stages[i]["op"] == "act":
            layer["act"] = stages[i]["fn"]
            i += 1
        layers.append(layer)
    return layers


class Program:
    """Flat layout + tower structure of an MLP actor-critic plan."""

    def __init__(self, plan: dict):
        if plan["compute_dtype"] not in ("float32", "bfloat16"):
            raise NotImplementedError(f"compute dtype {plan['compute_dtype']} is not compiled")
        self.bf16 = plan["compute_dtype"] == "bfloat16"
        if self.bf16 and plan.get("torso") is not None:
            raise NotImplementedError("a bf16 recurrent torso is not compiled")
        self.plan = plan
        L = FlatLayout()
        self.layout = L

        def dense(st, ld=None, w_region=None, b_region=None, col=0):
            fin, fout = st["in"], st["out"]
            if w_region is None:
                w_region = L.region(fin, ld or round_up(fout, 4))
            L.add_leaf(tuple(st["path"]) + ("kernel",), w_region.offset + col, (fin, fout), (w_region.ld, 1))
            if st.get("bias", True):
                if b_region is None:
                    b_region = L.region(1, w_region.ld)
                L.add_leaf(tuple(st["path"]) + ("bias",), b_region.offset + col, (fout,), (1,))
            return DenseSpec(tuple(st["path"]), fin, fout, w_region, b_region if st.get("bias", True) else None)

        def layer(g):
            d = dense(g["dense"])
            ln = None
            if g["ln"] is not None:
                F = g["dense"]["out"]
                sc, bi = L.region(1, F), L.region(1, F)
                L.add_leaf(tuple(g["ln"]["path"]) + ("scale",), sc.offset, (F,), (1,))
                L.add_leaf(tuple(g["ln"]["path"]) + ("bias",), bi.offset, (F,), (1,))
                ln = {"path": tuple(g["ln"]["path"]), "eps": g["ln"].get("eps", 1e-6), "scale": sc, "bias": bi}
            return LayerSpec(d, ln, g["act"])

        trunk = _group(plan["trunk"])
        actor = _group(plan["actor"])
        critic = _group(plan["critic"])
        if not actor or actor[-1]["ln"] is not None or actor[-1]["act"] is not None:
            raise NotImplementedError("the actor must end in a plain Dense")
        if not critic or critic[-1]["ln"] is not None or critic[-1]["act"] is not None:
            raise NotImplementedError("the critic must end in a plain Dense")
        actor_head, critic_head = actor[-1]["dense"], critic[-1]["dense"]
        actor, critic = actor[:-1], critic[:-1]
        if trunk and (actor or critic):
            raise NotImplementedError("a shared trunk followed by separate towers is not compiled")
        self.trunk = [layer(g) for g in trunk]
        self.gru = None
        if plan.get("torso") is not None:
            if actor or critic:
                raise NotImplementedError("a recurrent torso must feed plain Dense heads")
            self.gru = self._gru(L, plan["torso"])
        self.actor_layers = [layer(g) for g in actor]
        self.critic_layers = [layer(g) for g in critic]
        self.dist = plan["dist"]
        self.head_out = actor_head["out"]
        self.shared_head = not actor and not critic
        if self.shared_head:
            F = actor_head["in"]
            ldh = round_up(self.head_out + 1, 4)
            w = L.region(F, ldh)
            b = L.region(1, ldh)
            self.head_a = dense(actor_head, w_region=w, b_region=b, col=0)
            self.head_c = dense(critic_head, w_region=w, b_region=b, col=self.head_out)
        else:
            self.head_a = dense(actor_head)
            self.head_c = dense(critic_head)
        self.scale_region = None
        if self.dist["kind"] == "gaussian" and self.dist.get("scale") is not None:
            D = self.dist["dim"]
            self.scale_region = L.region(1, D)
            L.add_leaf(tuple(self.dist["scale"]), self.scale_region.offset, (D,), (1,))
        L.finish()

    @staticmethod
    def _gru(L: FlatLayout, t: dict) -> "GRUSpec":
        """flax GRUCell parameters as two side-by-side matrices: the input
        kernels [in, 3H] in column order (in, ir, iz) with their biases, and
        the recurrent kernels [H, 3H] in order (hr, hz, hn), plus hn's bias."""
        H, I = t["features"], t["in"]
        if H % 64:
            raise NotImplementedError("the GRU width must be a multiple of 64")
        base = tuple(t["path"])
        wi, bi = L.region(I, 3 * H), L.region(1, 3 * H)
        wh, bhn = L.region(H, 3 * H), L.region(1, H)
        for g, col in (("in", 0), ("ir", H), ("iz", 2 * H)):
            L.add_leaf(base + (g, "kernel"), wi.offset + col, (I, H), (3 * H, 1))
            L.add_leaf(base + (g, "bias"), bi.offset + col, (H,), (1,))
        for g, col in (("hr", 0), ("hz", H), ("hn", 2 * H)):
            L.add_leaf(base + (g, "kernel"), wh.offset + col, (H, H), (3 * H, 1))
        L.add_leaf(base + ("hn", "bias"), bhn.offset, (H,), (1,))
        return GRUSpec(base, I, H, wi, bi, wh, bhn)

    @property
    def action_dim(self) -> int:
        return self.dist["num"] if self.dist["kind"] == "categorical" else self.dist["dim"]


@dataclass
class GRUSpec:
    path: tuple
    fin: int
    H: int
    wi: Region
    bi: Region
    wh: Region
    bhn: Region


# --------------------------------------------------------------- buffers
def _splits(rows: int, m: int, n: int) -> int:
    """Row splits of a dW contraction over ``rows`` rows: at least 128 rows
    (four 32-deep stages) per split, and about 512 workgroups counted in
    128 x 128 tiles (2048-row minibatches: 16 splits, 31.4 -> 30.0 ms on the
    Gaussian update; 8 and 32 splits were both slower).  The 128 x 128-tile
    weight gradient of a 256 x 256 kernel over 32768 rows or more aims for
    256 workgroups instead (the Anakin minibatch's later layer: 64 splits,
    10.18 -> 10.12 ms per update; 128 splits 10.18, 32 splits 11.22)."""
    tiles = max(1, math.ceil(m / 128) * math.ceil(n / 128))
    target = 256 if m == 256 and n == 256 and rows >= 32768 else 512
    return max(1, min(max(1, rows // 128), math.ceil(target / tiles)))


@dataclass
class LayerBufs:
    spec: LayerSpec
    Y: torch.Tensor
    Z: torch.Tensor | None = None
    PRE: torch.Tensor | None = None
    mean: torch.Tensor | None = None
    rstd: torch.Tensor | None = None
    dY: torch.Tensor | None = None
    dZ: torch.Tensor | None = None
    wpart: torch.Tensor | None = None
    bpart: torch.Tensor | None = None
    lnpart: torch.Tensor | None = None
    splits: int = 1
    lnblocks: int = 0
    fpart: torch.Tensor | None = None
    dZ16: torch.Tensor | None = None
    Y16: torch.Tensor | None = None
    y32_unused: bool = False  # only the bf16 copy Y16 of this layer's output is read
    X16: torch.Tensor | None = None  # bf16 copy of a split-K first layer's input rows
    W16: torch.Tensor | None = None  # and of its kernel
    chain16: dict | None = None  # first layer of a bf16 chain group: the chain launch's pointer tables


class FlatState:
    """Device buffers of the parameters, gradient, Adam moments and count."""

    def __init__(self, program: Program, device):
        n = program.layout.size
        self.program = program
        self.device = device
        self.P = torch.zeros(n, dtype=torch.float32, device=device)
        self.G = torch.zeros(n, dtype=torch.float32, device=device)
        self.MU = torch.zeros(n, dtype=torch.float32, device=device)
        self.NU = torch.zeros(n, dtype=torch.float32, device=device)
        self.count = torch.zeros(1, dtype=torch.int32, device=device)
        # the compiled updates and rollout steps of this state (they live and
        # die with it)
        self.executors: dict = {}
        self.steppers: dict = {}

    def view(self, region: Region, col: int = 0) -> int:
        return self.P.data_ptr() + 4 * (region.offset + col)


def forward_bufs(spec: LayerSpec, rows: int, device) -> LayerBufs:
    """Forward-only buffers of one layer on ``rows`` rows: its output, and what
    the forward keeps (pre-LayerNorm values and statistics, pre-SiLU values)."""
    f32 = dict(dtype=torch.float32, device=device)
    b = LayerBufs(spec, Y=torch.zeros(rows, spec.ld, **f32))
    if spec.ln is not None:
        b.Z = torch.zeros(rows, spec.ld, **f32)
        b.mean = torch.zeros(rows, **f32)
        b.rstd = torch.zeros(rows, **f32)
    elif spec.act == "silu":
        b.PRE = torch.zeros(rows, spec.ld, **f32)
    return b


SPLIT_FWD_MIN_K = 1024  # a bf16 Dense reading an fp32 input this wide runs split-K


def split_forward_bufs(lb: LayerBufs, rows: int, device, bf16: bool) -> None:
    """Gives a group's first layer the fp32 partials of a split-K forward when
    it is a bf16 Dense with a long reduction over an fp32 input (the
    large-observation bootstrap and rollout step: few row tiles, so the
    reduction is what fills the chip)."""
    d = lb.spec.dense
    if not bf16 or d.fin < SPLIT_FWD_MIN_K or d.fin % 4 or lb.spec.ld % 4:
        return
    tiles = math.ceil(rows / 128) * math.ceil(lb.spec.ld / 128)
    S = max(1, min(math.ceil(256 / tiles), d.fin // 512, 16))
    # every split must own part of the reduction (64-element stages)
    while S > 1 and (S - 1) * (math.ceil(math.ceil(d.fin / S) / 64) * 64) >= d.fin:
        S -= 1
    if S > 1:
        lb.fpart = torch.zeros(S, rows, lb.spec.ld, dtype=torch.float32, device=device)
        if lb.spec.ld % 8 == 0:
            # bf16 copies of the input rows and of the kernel, so the GEMM takes
            # its direct global -> LDS copies (flax casts both to bf16 anyway)
            lb.X16 = torch.zeros(rows, (d.fin + 7) // 8 * 8, dtype=torch.int16, device=device)
            lb.W16 = torch.zeros(d.fin, d.w.ld, dtype=torch.int16, device=device)


def paired_tower_bufs(specs_a, specs_c, rows: int, device, ln_blocks: int | None = None,
                      grouped_dw: bool = False, fin0_pad: int = 0) -> tuple:
    """Training buffers of two towers of one shape (actor and critic, layer by
    layer): each kind of buffer of consecutive layers of one shape is one
    [layers, 2, ...] tensor, so the critic's buffer sits one fixed stride
    after the actor's at every depth (what a tower-batched launch addresses)
    and same-shape layers follow each other at that stride too (what a launch
    batched over depth addresses).  ``ln_blocks``: LayerNorm partial blocks
    of the backward that writes them (default: the row kernel's);
    ``grouped_dw``: the weight gradients past the first layer run as one
    launch batched over depth and towers.  ``fin0_pad``: the first layer's
    weight-gradient partials hold this many input rows (the width of a
    zero-padded copy of its input; the rows past the layer's own are never
    read)."""
    f32 = dict(dtype=torch.float32, device=device)
    L = len(specs_a)
    A = [LayerBufs(sa, Y=None) for sa in specs_a]
    C = [LayerBufs(sc, Y=None) for sc in specs_c]

    def alloc(attr, shapes):
        """Per-layer (actor, critic) views; runs of equal shapes share a tensor."""
        i = 0
        while i < L:
            if shapes[i] is None:
                i += 1
                continue
            j = i
            while j + 1 < L and shapes[j + 1] == shapes[i]:
                j += 1
            t = torch.zeros(j - i + 1, 2, *shapes[i], **f32)
            for k in range(i, j + 1):
                setattr(A[k], attr, t[k - i, 0])
                setattr(C[k], attr, t[k - i, 1])
            i = j + 1

    lib = _lib.load()
    ln = [s.ln is not None for s in specs_a]
    alloc("Y", [(rows, s.ld) for s in specs_a])
    alloc("dZ", [(rows, s.ld) for s in specs_a])
    alloc("Z", [(rows, s.ld) if ln[i] else None for i, s in enumerate(specs_a)])
    alloc("dY", [(rows, s.ld) if ln[i] else None for i, s in enumerate(specs_a)])
    alloc("mean", [(rows,) if ln[i] else None for i in range(L)])
    alloc("rstd", [(rows,) if ln[i] else None for i in range(L)])
    blocks = ln_blocks if ln_blocks else lib.ppo_layernorm_bwd_blocks(rows)
    alloc("lnpart", [(blocks, 2 * s.fout) if ln[i] else None for i, s in enumerate(specs_a)])
    alloc("PRE", [(rows, s.ld) if not ln[i] and s.act == "silu" else None for i, s in enumerate(specs_a)])
    for i, s in enumerate(specs_a):
        # batched over depth and towers in one launch that also finishes the
        # split-K sums (the last split of each tile reads the others'
        # partials back), fewer splits: half for the first layer, 3/8 for the
        # later ones (2048-row Gaussian minibatches: 8 and 6 splits, 5.08 M
        # samples/s, against 5.05 M with 16 and 8)
        sp = _splits(rows, s.dense.fin, s.ld)
        if grouped_dw:
            sp = sp // 2 if i == 0 else 3 * sp // 8
        A[i].splits = C[i].splits = max(1, sp)
        if ln[i]:
            A[i].lnblocks = C[i].lnblocks = blocks
    alloc("wpart", [(a.splits, max(s.dense.fin, fin0_pad) if i == 0 else s.dense.fin, s.ld)
                    for i, (a, s) in enumerate(zip(A, specs_a))])
    alloc("bpart", [(a.splits, s.ld) for a, s in zip(A, specs_a)])
    return A, C


def _tstride(a, c) -> int:
    """Element stride from tower 0's buffer (or pointer) to tower 1's."""
    pa = a if isinstance(a, int) else a.data_ptr()
    pc = c if isinstance(c, int) else c.data_ptr()
    assert (pc - pa) % 4 == 0
    return (pc - pa) // 4


class ForwardChain:
    """Issues the forward of Dense[+LayerNorm][+act] layer groups through the
    C ABI (fp32 MFMA, or the bf16 GEMMs with flax's casts for a bf16 network).
    The learner's executors and the rollout step share it."""

    def __init__(self, program: "Program", flat: "FlatState"):
        self._call = _lib.call
        self.prog = program
        self.bf16 = program.bf16
        self._ln_fwd = "ppo_layernorm_act_fwd_bf16" if self.bf16 else "ppo_layernorm_act_fwd_f32"
        self._ln_bwd = "ppo_layernorm_act_bwd_bf16" if self.bf16 else "ppo_layernorm_act_bwd_f32"
        self.flat = flat
        self.obs16 = False
        self.mb = -1
        self.inp: dict = {}

    @staticmethod
    def _f32_tile(a_layout: int, b_layout: int, M: int, K: int) -> int:
        """fp32 tile for a whole-minibatch contraction, measured per update:
        over 32768 rows or more (the Anakin minibatch) the 8-wave 256 x 128
        tile for forwards and 128 x 128 for the weight gradient of a 256-row
        kernel (11.43 -> 11.31 ms per update); at 16384 rows (the GRU
        workload) both were slower (17.8 -> 28.2 us on 16384 x 256 x 128,
        76 -> 90 us on its 256 x 768 dW), so below that the library's default
        (64 x 64).  The input cotangent (B = W^T) of a 32768-row minibatch
        also stays on 64 x 64: 10.18 ms per Anakin update against 10.54
        (256 x 128), 10.47 (128 x 128) and 10.51 (128 x 256)."""
        if a_layout == A_ROW and b_layout == B_KN and M >= 32768:
            return 9
        if a_layout == A_COL and M == 256 and K >= 32768:
            return 0
        return -1

    def _gemm(self, st, a_layout, b_layout, A, lda, rows, B, ldb, C, ldc, M, N, K, splits, stride, epi, bias, act,
              pre, aux, ldaux, bias_grad, tile):
        """One Dense contraction: fp32 MFMA, or for a bf16-compute network the
        bf16 MFMA GEMM with flax's casts (operands rounded to bf16 as read; the
        forward and input-cotangent results rounded to bf16; dW partials kept
        fp32 and rounded after their sum)."""
        if not self.bf16:
            if tile == -1:
                tile = self._f32_tile(a_layout, b_layout, M, K)
            self._call("ppo_gemm_f32", st, a_layout, b_layout, A, lda, rows, B, ldb, C, ldc, M, N, K, splits, stride,
                       epi, bias, act, pre, aux, ldaux, bias_grad, tile)
            return
        if pre is not None:
            raise NotImplementedError("a bf16 Dense with a SiLU activation and no LayerNorm is not compiled")
        round_out = 0 if a_layout == A_COL else 1
        self._call("ppo_gemm_bf16", st, a_layout, b_layout, A, lda, rows, B, ldb, C, ldc, M, N, K, splits, stride, epi,
                   bias, act, round_out, aux, ldaux, bias_grad, tile)

    def _reads_obs16(self, x, rows_idx, row0) -> bool:
        """True for the first layer of a minibatch pass over the observation
        (gathered rows of inputs["obs"]), which then reads the bf16 copy."""
        return self.obs16 and rows_idx is not None and row0 == 0 and x == self.inp["obs"]

    def _y16_input(self, layers, li, nrows, row0) -> bool:
        """True when layer li of a training group reads the bf16 output of
        layer li - 1 (minibatch passes of a bf16 network)."""
        return (li > 0 and row0 == 0 and nrows == self.mb and layers[li - 1].Y16 is not None
                and layers[li].spec.dense.w.ld % 8 == 0)

    def _ln_forward(self, st, lb, o, row0, nrows):
        s = lb.spec
        scale, bias = self.flat.view(s.ln["scale"]), self.flat.view(s.ln["bias"])
        if lb.Y16 is not None and row0 == 0 and nrows == self.mb:
            self._call("ppo_layernorm_act_fwd_bf16_out16", st, _p(lb.Z), s.ld, scale, bias,
                       None if lb.y32_unused else _p(lb.Y), s.ld,
                       _p(lb.Y16), s.ld, _p(lb.mean), _p(lb.rstd), nrows, s.fout, s.ln["eps"], _act(s.act))
        else:
            self._call(self._ln_fwd, st, _p(lb.Z) + o, s.ld, scale, bias, _p(lb.Y) + o, s.ld, _p(lb.mean) + 4 * row0,
                       _p(lb.rstd) + 4 * row0, nrows, s.fout, s.ln["eps"], _act(s.act))

    # The bf16 chain (ppo_mlp16_ln_fwd) runs a LayerNorm group's layers after
    # the first contraction in one launch, and its backward (ppo_mlp16_ln_bwd)
    # every LayerNorm backward and input cotangent of the group in another;
    # off, each layer has its own launches.
    CHAIN16 = True
    CHAIN16_BWD = True
    DW16_SIDE = True  # the chain group's later weight gradients beside the first layer's, on the side stream
    DW_SIDE = True    # fp32: a later layer's weight gradient beside its input cotangent, on the side stream
    # every weight gradient of the chain group in one launch (ppo_gemm_bf16s_dw_group):
    # the later layers' few tiles run beside the first layer's 198, with no
    # stream fork and join around them
    DW16_GROUP = True

    def _plan_chain16(self, group):
        """Pointer tables of the bf16 chain over ``group`` when it fits the
        chain: a first layer on the observation copy, then 512-wide Dense ->
        LayerNorm -> activation layers with biases, one activation and one
        epsilon; the later layers' kernels get packed operand images."""
        lib = _lib.load()
        if not (self.CHAIN16 and group and len(group) <= lib.ppo_mlp16_max_layers()
                and group[0].fpart is not None):
            return
        s0 = group[0].spec
        for i, lb in enumerate(group):
            s = lb.spec
            if (s.ln is None or s.fout != 512 or s.ld != 512 or s.dense.b is None or lb.Y16 is None
                    or _act(s.act) != _act(s0.act) or s.ln["eps"] != s0.ln["eps"]
                    or (i > 0 and (s.dense.fin != 512 or s.dense.w.ld != 512))):
                return
        view = self.flat.view
        arr = lambda xs: (ctypes.c_void_p * len(xs))(*xs)
        L = len(group)
        bwd = self.CHAIN16_BWD
        pk = torch.zeros(max(L - 1, 1), 2 if bwd else 1, 512 * 512, dtype=torch.int16, device=self.P16.device)
        if bwd:
            # the backward's LayerNorm gradient sums come in blocks of 32 rows
            blocks = lib.ppo_mlp16_ln_bwd_blocks(self.mb)
            for lb in group:
                if lb.lnpart.shape[0] < blocks:
                    lb.lnpart = torch.zeros(blocks, 2 * lb.spec.fout, dtype=torch.float32, device=self.P16.device)
                lb.lnblocks = blocks
        # with both chains, Z goes between them as bf16 (its values are bf16 numbers)
        z16 = [torch.zeros(self.mb, 512, dtype=torch.int16, device=self.P16.device) for _ in group] if bwd else None
        T = {"Wp": arr([None] + [_p(pk[l - 1, 0]) for l in range(1, L)]),
             "Wb": arr([None] + [_p(pk[l - 1, 1]) if bwd else None for l in range(1, L)]),
             "dZ16": arr([_p(lb.dZ16) for lb in group]),
             "part": arr([_p(lb.lnpart) for lb in group]),
             "b": arr([view(lb.spec.dense.b) for lb in group]),
             "g": arr([view(lb.spec.ln["scale"]) for lb in group]),
             "be": arr([view(lb.spec.ln["bias"]) for lb in group]),
             "Z": arr([_p(z) for z in z16] if bwd else [_p(lb.Z) for lb in group]),
             "Y": arr([None if lb.y32_unused else _p(lb.Y) for lb in group]),
             "Y16": arr([_p(lb.Y16) for lb in group]),
             "mean": arr([_p(lb.mean) for lb in group]),
             "rstd": arr([_p(lb.rstd) for lb in group])}
        addr = lambda a: ctypes.cast(a, ctypes.c_void_p).value
        c = {k: addr(v) for k, v in T.items()}
        c.update(keep=T, packed=pk, L=L, act=_act(s0.act), eps=float(s0.ln["eps"]), bwd=bwd, z16=int(bwd),
                 z16_bufs=z16)
        group[0].chain16 = c
        if L > 1:
            W = arr([self._view16(lb.spec.dense.w) for lb in group[1:]])
            F = arr([_p(pk[l, 0]) for l in range(L - 1)])
            B = arr([_p(pk[l, 1]) for l in range(L - 1)]) if bwd else None
            self._pack16_tables.append((L - 1, addr(W), addr(F), addr(B) if bwd else None, (W, F, B)))
            c["pack_F"] = addr(F)

    def _plan_chain16_head(self):
        """The shared head (heads.py:9-45) rides on the trunk chain's forward
        when it reads the trunk's 512-wide output: its packed operand image and
        the head output table of the chain launch."""
        prog = self.prog
        c = self.trunk[0].chain16 if self.trunk else None
        h = prog.head_a
        if (c is None or not prog.shared_head or self.fused or h.fin != 512 or h.b is None
                or h.w.ld > 256 or getattr(self, "HEAD", None) is None):
            return
        npad = (h.w.ld + 31) // 32 * 32
        hpk = torch.zeros(2, 512 * npad, dtype=torch.int16, device=self.P16.device)
        c.update(Wh=_p(hpk[0]), bh=self.flat.view(h.b), nh=h.w.ld, head=_p(self.HEAD), ldh=h.w.ld, head_pack=hpk,
                 head_npad=npad)
        if c["bwd"] and npad <= 64:
            # the backward chain also takes the head's input cotangent over,
            # and the head's dW reads the bf16 output: the chain's fp32 one is
            # not needed
            c.update(Whb=_p(hpk[1]))
            c["keep"]["Y"][c["L"] - 1] = None
            if self.DW16_GROUP and c["L"] < 8 and self.head_splits == self.HEAD16_SPLITS:
                # the chain leaves the rounded head cotangents as bf16, and the
                # head's dW joins the trunk's grouped dW launch
                ld16 = (h.w.ld + 7) // 8 * 8
                self.DHEAD16 = torch.zeros(self.mb, ld16, dtype=torch.int16, device=self.P16.device)
                c.update(dhead16=(_p(self.DHEAD16), ld16))

    def _pack16(self, st):
        """Packed operand images of the bf16 chains' kernels from the bf16
        parameter image (after each write of the image)."""
        c = self.trunk[0].chain16 if self.trunk else None
        head = c is not None and c.get("Wh")
        h = self.prog.head_a
        packed_head = False
        for n, W, F, B, _ in self._pack16_tables:
            # the trunk's head rides in the same launch
            hargs = (None, 0, 0, 0, None, None)
            if head and F == c.get("pack_F"):
                hargs = (self._view16(h.w), h.w.ld, h.w.ld, c["head_npad"], c["Wh"], c.get("Whb"))
                packed_head = True
            self._call("ppo_pack_bf16_operands", st, n, W, 512, 512, 512, F, B, *hargs)
        if head and not packed_head:
            self._call("ppo_pack_bf16_operand_padded", st, self._view16(h.w), h.w.ld, 512, h.w.ld, c["head_npad"],
                       c["Wh"], c.get("Whb"))

    def _view16(self, region: Region) -> int:
        """Address of a parameter region in the bf16 parameter image."""
        return _p(self.P16) + 2 * region.offset

    def _fwd_layers(self, st, layers, x, ldx, rows_idx, nrows, row0=0):
        """Forward of Dense[+LayerNorm][+act] layers on nrows rows, writing
        each layer's buffers from row ``row0`` on."""
        for li, lb in enumerate(layers):
            s = lb.spec
            d = s.dense
            W = self.flat.view(d.w)
            Bb = self.flat.view(d.b) if d.b is not None else None
            o = 4 * row0 * s.ld
            if li == 0 and self._reads_obs16(x, rows_idx, row0):
                dst = lb.Z if s.ln is not None else lb.Y
                self._call("ppo_gemm_bf16s", st, A_ROW, B_KN, 1, 1, _p(self.OBS16), self.ldo16, rows_idx,
                           self._view16(d.w), d.w.ld, _p(lb.fpart), s.ld, nrows, s.ld, d.fin, self.FWD16_SPLITS,
                           nrows * s.ld, EPI_STORE, None, 0, 0, None, 0, None, self.FWD16_TILE)
                c = lb.chain16
                if c is not None and nrows == self.mb and row0 == 0:
                    # the rest of the group in one launch from the split partials
                    self._call("ppo_mlp16_ln_fwd", st, c["L"], _p(lb.fpart), s.ld, nrows * s.ld,
                               self.FWD16_SPLITS, nrows, c["Wp"], c["b"], c["g"], c["be"], c["Z"], c["Y"],
                               c["Y16"], s.ld, c["mean"], c["rstd"], c["eps"], c["act"], c.get("Wh"), c.get("bh"),
                               c.get("nh", 0), c.get("head"), c.get("ldh", 0), c["z16"])
                    top = layers[-1]
                    return _p(top.Y), top.spec.ld, None
                self._call("ppo_splits_bias_act_bf16", st, _p(lb.fpart), s.ld, nrows * s.ld, self.FWD16_SPLITS, Bb,
                           _act(s.act) if s.ln is None else 0, _p(dst), s.ld, nrows, s.ld)
                if s.ln is not None:
                    self._ln_forward(st, lb, o, row0, nrows)
            elif (li == 0 and lb.fpart is not None and rows_idx is None and row0 == 0 and self.bf16
                  and x % 16 == 0 and ldx % 4 == 0 and nrows <= lb.fpart.shape[1]):
                # bf16 Dense on an fp32 input: split-K partials on the pipelined
                # GEMM (operands rounded to bf16 as staged), summed in split
                # order with flax's bf16 bias add and activation
                S = lb.fpart.shape[0]
                dst = lb.Z if s.ln is not None else lb.Y
                if lb.X16 is not None and nrows <= lb.X16.shape[0]:
                    ld16 = lb.X16.shape[1]
                    self._call("ppo_cast_bf16_2d", st, x, ldx, _p(lb.X16), ld16, nrows, d.fin)
                    self._call("ppo_cast_bf16", st, W, _p(lb.W16), d.fin * d.w.ld)
                    self._call("ppo_gemm_bf16s", st, A_ROW, B_KN, 1, 1, _p(lb.X16), ld16, None, _p(lb.W16), d.w.ld,
                               _p(lb.fpart), s.ld, nrows, s.ld, d.fin, S, lb.fpart.shape[1] * s.ld, EPI_STORE, None,
                               0, 0, None, 0, None, 1)
                else:
                    self._call("ppo_gemm_bf16s", st, A_ROW, B_KN, 0, 0, x, ldx, None, W, d.w.ld, _p(lb.fpart),
                               s.ld, nrows, s.ld, d.fin, S, lb.fpart.shape[1] * s.ld, EPI_STORE, None, 0, 0, None,
                               0, None, -1)
                self._call("ppo_splits_bias_act_bf16", st, _p(lb.fpart), s.ld, lb.fpart.shape[1] * s.ld, S, Bb,
                           _act(s.act) if s.ln is None else 0, _p(dst), s.ld, nrows, s.ld)
                if s.ln is not None:
                    self._ln_forward(st, lb, o, row0, nrows)
            elif self._y16_input(layers, li, nrows, row0):
                prev = layers[li - 1]
                dst = lb.Z if s.ln is not None else lb.Y
                self._call("ppo_gemm_bf16s", st, A_ROW, B_KN, 1, 1, _p(prev.Y16), prev.spec.ld, None,
                           self._view16(d.w), d.w.ld, _p(dst), s.ld, nrows, s.ld, d.fin, 1, 0, EPI_BIAS_ACT, Bb,
                           _act(s.act) if s.ln is None else 0, 1, None, 0, None, -1)
                if s.ln is not None:
                    self._ln_forward(st, lb, o, row0, nrows)
            elif s.ln is not None and not self.bf16 and s.fout == 256 and s.ld == 256:
                # Dense -> LayerNorm -> activation in one launch (16 rows x 256 columns per workgroup)
                self._call("ppo_gemm_ln_act_fwd_f32", st, x, ldx, rows_idx, W, d.w.ld, Bb,
                           self.flat.view(s.ln["scale"]), self.flat.view(s.ln["bias"]), _p(lb.Z) + o, s.ld,
                           _p(lb.Y) + o, s.ld, _p(lb.mean) + 4 * row0, _p(lb.rstd) + 4 * row0, nrows, d.fin, s.fout,
                           s.ln["eps"], _act(s.act))
            elif s.ln is not None:
                self._gemm(st, A_ROW, B_KN, x, ldx, rows_idx, W, d.w.ld, _p(lb.Z) + o, s.ld, nrows,
                          s.ld, d.fin, 1, 0, EPI_BIAS_ACT, Bb, 0, None, None, 0, None, -1)
                self._ln_forward(st, lb, o, row0, nrows)
            else:
                pre = _p(lb.PRE) + o if lb.PRE is not None else None
                self._gemm(st, A_ROW, B_KN, x, ldx, rows_idx, W, d.w.ld, _p(lb.Y) + o, s.ld, nrows,
                          s.ld, d.fin, 1, 0, EPI_BIAS_ACT, Bb, _act(s.act), pre, None, 0, None, -1)
            x, ldx, rows_idx = _p(lb.Y) + o, s.ld, None
        return x, ldx, rows_idx


class MLPExecutor(ForwardChain):
    """One compiled PPO.update for fixed (T, N, obs, minibatches, epochs)."""

    FWD16_SPLITS = 2  # K splits of the bf16 first-layer forward (256 workgroups of 256 x 128 at 8192 x 512)
    FWD16_TILE = 0    # 256 x 128 tiles, three-stage ring (8192 x 512 x 8268 with gathered rows: 96.9 -> 85.4 us
    #                   against 128 x 128 tiles, two resident per CU, measured with cold rows)
    DW16_SPLITS = 3   # row splits of the bf16 first-layer dW (with 256 x 256 tiles: 198 workgroups at 8268 x 512)
    DW16_TILE = 2     # 256 x 256 tiles for the bf16 first-layer dW
    # row splits of a bf16 dW between two LayerNorm layers: with the chains these
    # run in the first layer's dW launch, where 3 splits (12 workgroups of
    # 256 x 256 each) take as long as the first layer's workgroups; on the side
    # stream 4 splits of 128 x 128 tiles finished inside the first layer's dW
    # (large-observation update 14.70 -> 14.2-14.3 ms from 16 splits; 2 splits
    # 15.0, 1 split 18.5)
    DW16_SPLITS_INNER = 3
    # row splits of the shared head's dW in a bf16 network: in the grouped dW
    # launch its 2 x 4 workgroups of 2048 rows finish inside the first layer's
    HEAD16_SPLITS = 4

    def __init__(self, program: Program, flat: FlatState, cfg, chain, T: int, N: int):
        if program.gru is not None and type(self) is MLPExecutor:
            raise TypeError("a recurrent program runs on RecurrentExecutor")
        ForwardChain.__init__(self, program, flat)
        self.cfg = cfg
        self.chain = chain
        self.T, self.N = T, N
        self.B = T * N
        self.E = int(cfg.update_epochs)
        self.M = int(cfg.num_minibatches)
        self.perm_n = self._perm_size()
        if self.perm_n % self.M:
            raise ValueError(f"{self.perm_n} permuted items are not divisible into {self.M} minibatches")
        self.mb = self.B // self.M
        dev = flat.device
        f32 = dict(dtype=torch.float32, device=dev)
        self.obs_dim = program.plan["obs_dim"]
        mb = self.mb

        def layer_bufs(spec: LayerSpec, rows: int, train: bool) -> LayerBufs:
            ld = spec.ld
            b = forward_bufs(spec, rows, dev)
            if train:
                b.dZ = torch.zeros(rows, ld, **f32)
                if spec.ln is not None:
                    b.dY = torch.zeros(rows, ld, **f32)
                    b.lnblocks = _lib.load().ppo_layernorm_bwd_blocks(rows)
                    b.lnpart = torch.zeros(b.lnblocks, 2 * spec.fout, **f32)
                b.splits = _splits(rows, spec.dense.fin, ld)
                b.wpart = torch.zeros(b.splits, spec.dense.fin, ld, **f32)
                b.bpart = torch.zeros(b.splits, ld, **f32)
            return b

        self.trunk = [layer_bufs(s, mb, True) for s in program.trunk]
        # an actor and a critic tower of one shape (flax's ActorCritic with
        # separate torsos) run each depth's forward, LayerNorm backward, dW
        # and input-cotangent contraction for both towers in one launch
        self.pair = self._pair_stride(program)
        # towers of 256-wide LayerNorm layers (one activation, one epsilon)
        # run each direction of the whole torso chain in one launch
        self.chain_ln = bool(self.pair) and self.CHAIN and self._chainable(program.actor_layers)
        # observation rows whose width is not a multiple of four: a zero-padded
        # copy per update lets the first layer's weight gradient run on the
        # copy-fed GEMM over the padded width (the Gaussian workload's 87
        # features: 10.2 us per step on the register-staged kernel)
        fin0 = program.actor_layers[0].dense.fin if program.actor_layers else 0
        self.obs_pad = (fin0 + 3) // 4 * 4 if self.chain_ln and fin0 % 4 != 0 and fin0 == self.obs_dim else 0
        if self.pair:
            lnb = _lib.load().ppo_mlp_ln_bwd_blocks(mb) if self.chain_ln else None
            self.actor, self.critic = paired_tower_bufs(program.actor_layers, program.critic_layers, mb, dev, lnb,
                                                        grouped_dw=self.chain_ln, fin0_pad=self.obs_pad)
        else:
            self.actor = [layer_bufs(s, mb, True) for s in program.actor_layers]
            self.critic = [layer_bufs(s, mb, True) for s in program.critic_layers]
        # bf16 network: the first Dense of each torso group contracts the bf16
        # observation copy with the bf16 image of the parameters on the
        # pipelined GEMM (forward split over K, dW over rows)
        firsts = [g[0] for g in (self.trunk, self.actor, self.critic) if g]
        self.obs16 = (self.bf16 and program.gru is None and self.obs_dim % 4 == 0 and bool(firsts)
                      and all(lb.spec.ld % 8 == 0 and lb.spec.dense.w.ld % 8 == 0 for lb in firsts))
        if self.obs_pad:
            self.OBSP = torch.zeros(self.B, self.obs_pad, dtype=torch.float32, device=dev)
        if self.obs16:
            i16 = dict(dtype=torch.int16, device=dev)
            self.ldo16 = (self.obs_dim + 7) // 8 * 8
            self.OBS16 = torch.zeros(self.B, self.ldo16, **i16)
            self.P16 = torch.zeros(flat.P.numel(), **i16)
            for lb in firsts:
                d = lb.spec.dense
                lb.splits = self.DW16_SPLITS
                lb.wpart = torch.zeros(lb.splits, d.fin, lb.spec.ld, **f32)
                lb.bpart = torch.zeros(lb.splits, lb.spec.ld, **f32)
                lb.fpart = torch.zeros(self.FWD16_SPLITS, mb, lb.spec.ld, **f32)
                if lb.spec.ln is not None:
                    lb.dZ16 = torch.zeros(mb, lb.spec.ld, **i16)
            # the LayerNorm layers also keep their output and take their
            # cotangent as bf16, so every torso contraction has bf16 operands
            for group in (self.trunk, self.actor, self.critic):
                for li, lb in enumerate(group):
                    if lb.spec.ln is None:
                        continue
                    lb.Y16 = torch.zeros(mb, lb.spec.ld, **i16)
                    if lb.dZ16 is None:
                        lb.dZ16 = torch.zeros(mb, lb.spec.ld, **i16)
                    # the next Dense reads (forward and dW) only the bf16 copy
                    lb.y32_unused = li + 1 < len(group) and group[li + 1].spec.dense.w.ld % 8 == 0
                    if li > 0 and group[li - 1].spec.ln is not None:
                        d = lb.spec.dense
                        lb.splits = self.DW16_SPLITS_INNER
                        lb.wpart = torch.zeros(lb.splits, d.fin, lb.spec.ld, **f32)
                        lb.bpart = torch.zeros(lb.splits, lb.spec.ld, **f32)
        self._pack16_tables = []
        if self.obs16:
            for group in (self.trunk, self.actor, self.critic):
                self._plan_chain16(group)
        self.boot_layers = [layer_bufs(s, self._boot_rows(), False) for s in
                            (program.trunk if program.shared_head else program.critic_layers)]
        if self.boot_layers and program.gru is None:
            split_forward_bufs(self.boot_layers[0], self._boot_rows(), dev, self.bf16)
        if self.chain_ln:
            L = len(self.actor)
            self.WT = torch.zeros(max(L - 1, 1), 2, 256, 256, **f32)
            self._chain_tables()
        ha, hc = program.head_a, program.head_c
        lib = _lib.load()
        self.fused = self._can_fuse(program)
        if self.fused:
            hb = lib.ppo_head_loss_blocks(mb)
            self.head_blocks = hb
        if self.fused and program.shared_head:
            self.HWPART = torch.zeros(hb, ha.fin, ha.w.ld, **f32)
            self.HBPART = torch.zeros(hb, ha.w.ld, **f32)
            self.head_splits = hb
            self.HEADB = torch.zeros(N, ha.w.ld, **f32)
        elif self.fused:
            self.HAWPART = torch.zeros(hb, ha.fin, ha.w.ld, **f32)
            self.HABPART = torch.zeros(hb, ha.w.ld, **f32)
            self.HCWPART = torch.zeros(hb, hc.fin, hc.w.ld, **f32)
            self.HCBPART = torch.zeros(hb, hc.w.ld, **f32)
            self.ha_splits = self.hc_splits = hb
            self.HEADB = torch.zeros(N, hc.w.ld, **f32)
        elif program.shared_head:
            self.HEAD = torch.zeros(mb, ha.w.ld, **f32)
            self.DHEAD = torch.zeros(mb, ha.w.ld, **f32)
            # bf16 networks: the head's dW may run in the trunk's grouped dW
            # launch, and both backward paths keep the same split boundaries
            self.head_splits = self.HEAD16_SPLITS if self.obs16 else _splits(mb, ha.fin, ha.w.ld)
            self.HWPART = torch.zeros(self.head_splits, ha.fin, ha.w.ld, **f32)
            self.HBPART = torch.zeros(self.head_splits, ha.w.ld, **f32)
            self.HEADB = torch.zeros(N, ha.w.ld, **f32)
        else:
            self.HA = torch.zeros(mb, ha.w.ld, **f32)
            self.DHA = torch.zeros(mb, ha.w.ld, **f32)
            self.HC = torch.zeros(mb, hc.w.ld, **f32)
            self.DHC = torch.zeros(mb, hc.w.ld, **f32)
            self.ha_splits = _splits(mb, ha.fin, ha.w.ld)
            self.hc_splits = _splits(mb, hc.fin, hc.w.ld)
            self.HAWPART = torch.zeros(self.ha_splits, ha.fin, ha.w.ld, **f32)
            self.HABPART = torch.zeros(self.ha_splits, ha.w.ld, **f32)
            self.HCWPART = torch.zeros(self.hc_splits, hc.fin, hc.w.ld, **f32)
            self.HCBPART = torch.zeros(self.hc_splits, hc.w.ld, **f32)
            self.HEADB = torch.zeros(N, hc.w.ld, **f32)
        self._plan_chain16_head()
        self.loss_blocks = self.head_blocks if self.fused else lib.ppo_loss_blocks(mb)
        self.nstat = lib.ppo_loss_stat_count()
        # loss statistics of every step, finalized into LOGS once per update
        self.STATS = torch.zeros(self.E * self.M, self.loss_blocks, self.nstat, dtype=torch.float64, device=dev)
        self.DSCALE = (torch.zeros(self.loss_blocks, program.dist["dim"], **f32)
                       if program.scale_region is not None else None)
        self.LOGS = torch.zeros(self.E * self.M, 9, **f32)
        self.BOOT = torch.zeros(N, **f32)
        self.ADV = torch.zeros(self.B, **f32)
        self.RET = torch.zeros(self.B, **f32)
        # the fused loss's per-sample inputs as 32-byte records (see _pack_samples)
        self.REC = torch.zeros(self.B, 8, **f32) if self.RECORDS and self.fused else None
        self.PERM = torch.zeros(self.E, self.perm_n, dtype=torch.int32, device=dev)
        ws = lib.ppo_epoch_permutations_workspace(self.E, self.perm_n)
        self.PERM_WS = torch.zeros(ws, dtype=torch.uint8, device=dev)
        self.KEY = torch.zeros(2, dtype=torch.int32, device=dev)
        self.NORM_WS = torch.zeros(max(1, lib.ppo_normalize_workspace(self.B)), dtype=torch.uint8, device=dev)
        self._alloc_extra()
        self._build_reduce_tables()
        # separate actor and critic towers run their chains on two streams
        self.side = torch.cuda.Stream(device=dev) if torch.device(dev).type == "cuda" else None
        self._recording = False
        self._ev_fork = self._ev_join = None
        if self.side is not None:
            evs = []
            for _ in range(2):
                h = ctypes.c_void_p()
                self._call("ppo_event_create", ctypes.byref(h))
                evs.append(h.value)
            self._ev_fork, self._ev_join = evs
            # destroyed when the executor is collected, or at interpreter exit
            # (before module teardown) with the destroy function held here
            weakref.finalize(self, _destroy_events, lib.ppo_event_destroy, tuple(evs))

    def _alloc_extra(self):
        """Buffers a subclass adds before the gradient tables are built."""

    def _extra_segments(self, G: int) -> list:
        """Gradient segments (dst, src, count, part_stride, nparts, flags) a subclass adds."""
        return []

    @staticmethod
    def _can_fuse(program: Program) -> bool:
        """The fused head + loss kernel applies when the heads read torso
        features (not the raw observation) of one width <= 512 and the actor
        head has at most 16 outputs (plus the value column when shared)."""
        lib = _lib.load()
        ha, hc = program.head_a, program.head_c
        if program.bf16:
            return False
        if program.shared_head:
            if not program.trunk and program.gru is None:
                return False
            na = program.head_out + 1
        else:
            if not program.actor_layers or not program.critic_layers or ha.fin != hc.fin:
                return False
            na = program.head_out
        return (na <= lib.ppo_head_loss_max_outputs() and ha.fin <= lib.ppo_head_loss_max_features()
                and ha.fin % 16 == 0)

    CHAIN = True  # paired LayerNorm towers run whole-chain launches

    @staticmethod
    def _chainable(layers) -> bool:
        """Layers the whole-chain launches take: 1 to ppo_mlp_chain_max_layers()
        Dense(256) -> LayerNorm -> activation layers of one activation and
        epsilon, 256-element rows."""
        if not layers or len(layers) > _lib.load().ppo_mlp_chain_max_layers():
            return False
        s0 = layers[0]
        return all(s.ln is not None and s.fout == 256 and s.ld == 256 and s.act == s0.act
                   and s.ln["eps"] == s0.ln["eps"] and s.dense.w.ld == 256 for s in layers)

    def _chain_tables(self):
        """Per-layer pointer tables of the chain launches (ctypes arrays kept
        alive on the executor; the pointers are fixed for its lifetime)."""
        view = self.flat.view
        A, C = self.actor, self.critic
        specs = [lb.spec for lb in A]
        L = len(A)
        arr = lambda xs: (ctypes.c_void_p * len(xs))(*xs)
        T = {}
        T["W"] = arr([view(s.dense.w) for s in specs])
        T["b"] = arr([view(s.dense.b) if s.dense.b is not None else None for s in specs])
        T["g"] = arr([view(s.ln["scale"]) for s in specs])
        T["be"] = arr([view(s.ln["bias"]) for s in specs])
        T["Z"] = arr([_p(lb.Z) for lb in A])
        T["Y"] = arr([_p(lb.Y) for lb in A])
        T["mean"] = arr([_p(lb.mean) for lb in A])
        T["rstd"] = arr([_p(lb.rstd) for lb in A])
        T["dZ"] = arr([_p(lb.dZ) for lb in A])
        T["part"] = arr([_p(lb.lnpart) for lb in A])
        # the forward writes layer l >= 1's kernel transposed into WT[l - 1, tower]
        T["WT"] = arr([None] + [_p(self.WT[l - 1, 0]) for l in range(1, L)])
        boot = self.boot_layers
        cspecs = [lb.spec for lb in boot]
        T["bW"] = arr([view(s.dense.w) for s in cspecs])
        T["bb"] = arr([view(s.dense.b) if s.dense.b is not None else None for s in cspecs])
        T["bg"] = arr([view(s.ln["scale"]) for s in cspecs])
        T["bbe"] = arr([view(s.ln["bias"]) for s in cspecs])
        T["bZ"] = arr([_p(lb.Z) for lb in boot])
        T["bY"] = arr([_p(lb.Y) for lb in boot])
        T["bmean"] = arr([_p(lb.mean) for lb in boot])
        T["brstd"] = arr([_p(lb.rstd) for lb in boot])
        addr = lambda a: ctypes.cast(a, ctypes.c_void_p).value
        self._chain_keep = T
        self._chain = {k: (addr(v) if isinstance(v, ctypes.Array) else v) for k, v in T.items()}
        s0 = specs[0]
        self._chain_act, self._chain_eps = _act(s0.act), float(s0.ln["eps"])
        self._dw_groups = self._plan_dw_groups()
        self._chain_rs = _tstride(A[0].Y, C[0].Y)
        self._chain_ss = _tstride(A[0].mean, C[0].mean)
        self._chain_ps = _tstride(A[0].lnpart, C[0].lnpart)
        assert all(_tstride(a.Z, c.Z) == self._chain_rs == _tstride(a.dZ, c.dZ) == _tstride(a.Y, c.Y)
                   and _tstride(a.mean, c.mean) == self._chain_ss == _tstride(a.rstd, c.rstd)
                   and _tstride(a.lnpart, c.lnpart) == self._chain_ps for a, c in zip(A, C))

    # the paired towers' weight gradients in one ppo_gemm_f32_dw_group launch
    # (off: one launch for the first layers, one for the rest)
    PAIR_DW_GROUP = True

    # the paired towers' weight gradients finish their split-K sums in their
    # grouped launch (no gradient-reduce launch for them); the split counts
    # that launch supports
    DW_FINAL = True
    FINAL_SPLITS = (1, 2, 3, 4, 6, 8, 12, 16, 32, 64)

    def _first_dw_final(self, st, layers, x, ldx, ridx) -> bool:
        """The shared trunk's first-layer weight gradient as a one-problem
        ppo_gemm_f32_dw_group_final launch that also assembles every other
        leaf's gradient (the optimizer step then skips the reduce); False when
        the trunk does not take it (the caller runs the plain GEMM)."""
        fin = self.dw_final
        if fin is None or not fin.get("first") or layers is not self.trunk or x % 16 or ldx % 4:
            return False
        g = self.__dict__.get("_ffa")
        if g is None or g["x"] != (x, ldx):
            # host argument arrays, kept (a recorded launch is replayed from them); the
            # gather indices are set per call in rows[0]
            lb = layers[0]
            s, d = lb.spec, lb.spec.dense
            G = self.flat.G.data_ptr()
            vp = lambda v: (ctypes.c_void_p * 1)(v)
            arrs = [vp(x), (ctypes.c_int64 * 1)(ldx), vp(None), vp(_p(lb.dZ)), (ctypes.c_int64 * 1)(s.ld),
                    vp(_p(lb.wpart)), (ctypes.c_int64 * 1)(s.ld), (ctypes.c_int * 1)(d.fin), (ctypes.c_int * 1)(s.ld),
                    (ctypes.c_int * 1)(self.mb), (ctypes.c_int * 1)(fin["first"]), (ctypes.c_int64 * 1)(d.fin * s.ld),
                    vp(_p(lb.bpart)), vp(G + 4 * d.w.offset), (ctypes.c_int64 * 1)(d.w.ld), (ctypes.c_int * 1)(d.fin),
                    vp(G + 4 * d.b.offset if d.b is not None else None)]
            g = self._ffa = {"x": (x, ldx), "arrs": arrs, "rows": arrs[2],
                             "args": [ctypes.addressof(a) for a in arrs]}
        g["rows"][0] = ridx
        self._call("ppo_gemm_f32_dw_group_final", st, 1, *g["args"], _p(fin["CNT"]), _p(fin["SUMSQ"]),
                   _p(fin["SEGS"]), _p(fin["CHUNKS"]), fin["nchunks"], fin["nfew"], fin["nwide"])
        self._dw_finished = True
        return True

    def _pair_dw_shapes(self):
        """(M, N, splits) of every problem of the paired towers' grouped
        weight-gradient launch, in its order (layer-major, actor then
        critic), or None when the towers do not take that launch."""
        A, C = self.actor, self.critic
        if not self.PAIR_DW_GROUP or not self.chain_ln or 2 * len(A) > 8:
            return None
        fin0 = self.obs_pad if self.obs_pad else A[0].spec.dense.fin
        return [(fin0 if i == 0 else lb.spec.dense.fin, lb.spec.ld, lb.splits)
                for i in range(len(A)) for lb in (A[i], C[i])]

    def _pair_dw_group(self, x0, ldx0):
        """Host argument arrays of ppo_gemm_f32_dw_group over every weight
        gradient of the paired towers (layer-major, actor then critic; the
        first layers read the observation rows, or their zero-padded copy,
        through the minibatch's gather indices, set per call in rows[0] and
        rows[1]), or None when a problem does not fit the copy-fed kernel."""
        A, C = self.actor, self.critic
        if not self.PAIR_DW_GROUP or 2 * len(A) > 8:
            return None
        g = getattr(self, "_dwg", None)
        if g is not None and g["x0"] == (x0, ldx0):
            return g if g["args"] else None
        x, ldx, fin0 = (_p(self.OBSP), self.obs_pad, self.obs_pad) if self.obs_pad else (x0, ldx0, A[0].spec.dense.fin)
        probs = []  # (A, lda, B, ldb, C, ldc, M, N, splits, bias_grad)
        for i in range(len(A)):
            for lb, prev in ((A[i], A[i - 1] if i else None), (C[i], C[i - 1] if i else None)):
                s = lb.spec
                a, lda, M = (x, ldx, fin0) if i == 0 else (_p(prev.Y), prev.spec.ld, s.dense.fin)
                probs.append((a, lda, _p(lb.dZ), s.ld, _p(lb.wpart), s.ld, M, s.ld, lb.splits, _p(lb.bpart)))
        fits = all(a % 16 == 0 and lda % 4 == 0 and M % 4 == 0 and N % 4 == 0 and b % 16 == 0 and ldb % 4 == 0
                   and (i >= 2 or -(-self.mb // sp) <= 2048)
                   for i, (a, lda, b, ldb, _, _, M, N, sp, _) in enumerate(probs))
        g = {"x0": (x0, ldx0), "args": None}
        self._dwg = g
        if not fits:
            return None
        L = len(probs)
        vp = lambda xs: (ctypes.c_void_p * L)(*xs)
        i64 = lambda xs: (ctypes.c_int64 * L)(*xs)
        i32 = lambda xs: (ctypes.c_int * L)(*xs)
        col = lambda j: [p[j] for p in probs]
        g.update({
            "A": vp(col(0)), "lda": i64(col(1)), "rows": vp([None] * L), "B": vp(col(2)), "ldb": i64(col(3)),
            "C": vp(col(4)), "ldc": i64(col(5)), "M": i32(col(6)), "N": i32(col(7)), "K": i32([self.mb] * L),
            "splits": i32(col(8)), "stride": i64([p[6] * p[5] for p in probs]), "bias_grad": vp(col(9)),
            "count": L,
        })
        order = ("A", "lda", "rows", "B", "ldb", "C", "ldc", "M", "N", "K", "splits", "stride", "bias_grad")
        g["args"] = [ctypes.addressof(g[k]) for k in order]
        fin = self.dw_final
        if fin is not None:
            # the final gradients: problem order as above
            G = self.flat.G.data_ptr()
            lbs = [lb for i in range(len(A)) for lb in (A[i], C[i])]
            g.update({
                "G": vp([G + 4 * lb.spec.dense.w.offset for lb in lbs]),
                "ldg": i64([lb.spec.dense.w.ld for lb in lbs]),
                "g_rows": i32([lb.spec.dense.fin for lb in lbs]),
                "Gb": vp([G + 4 * lb.spec.dense.b.offset if lb.spec.dense.b is not None else None for lb in lbs]),
            })
            g["final_args"] = g["args"] + [ctypes.addressof(g[k]) for k in ("G", "ldg", "g_rows", "Gb")] + [
                _p(fin["CNT"]), _p(fin["SUMSQ"]), _p(fin["SEGS"]), _p(fin["CHUNKS"]), fin["nchunks"], fin["nfew"],
                fin["nwide"]]
        return g

    def _plan_dw_groups(self) -> list:
        """The weight-gradient contractions of the paired towers as batched
        launches: layer 0 of both towers (the gathered observation rows
        shared), then every later layer of both towers in one launch when
        their operands sit at one stride from problem to problem
        (layer-major, tower-minor), else layer by layer.  Entries:
        (first layer, problems, input stride)."""
        A, C = self.actor, self.critic
        L = len(A)
        groups = [(0, 2, 0)]
        probs = [(i, t) for i in range(1, L) for t in range(2)]
        if len(probs) >= 2 and len(probs) <= 8:
            lbs = lambda i, t: (A if t == 0 else C)[i]
            shapes = {(lbs(i, t).spec.dense.fin, lbs(i, t).spec.ld, lbs(i, t).splits) for i, t in probs}
            ptrs = [(_p(lbs(i - 1, t).Y), _p(lbs(i, t).dZ), _p(lbs(i, t).wpart), _p(lbs(i, t).bpart))
                    for i, t in probs]
            steps = {tuple(b - a for a, b in zip(ptrs[k], ptrs[k + 1])) for k in range(len(ptrs) - 1)}
            if len(shapes) == 1 and len(steps) == 1:
                groups.append((1, len(probs), (ptrs[1][0] - ptrs[0][0]) // 4))
                return groups
        groups += [(i, 2, _tstride(A[i - 1].Y, C[i - 1].Y)) for i in range(1, L)]
        return groups

    def _pair_stride(self, program: Program) -> int:
        """Element offset from every parameter region of the actor tower to the
        same region of the critic tower when the two towers have one shape
        (fp32, fused head loss) and can share launches; else 0."""
        A, C = program.actor_layers, program.critic_layers
        if (self.bf16 or program.gru is not None or program.shared_head or not A or len(A) != len(C)
                or not self._can_fuse(program)):
            return 0
        D = None
        for a, c in zip(A, C):
            shape = lambda s: (s.dense.fin, s.fout, s.ld, s.act, s.dense.b is None, s.ln is None,
                               s.ln["eps"] if s.ln is not None else None)
            if shape(a) != shape(c):
                return 0
            if a.ln is not None and (a.fout != 256 or a.ld != 256):
                return 0   # LayerNorm layers run the fused 256-wide Dense + LayerNorm forward
            regions = [(a.dense.w, c.dense.w)]
            if a.dense.b is not None:
                regions.append((a.dense.b, c.dense.b))
            if a.ln is not None:
                regions += [(a.ln["scale"], c.ln["scale"]), (a.ln["bias"], c.ln["bias"])]
            for ra, rc in regions:
                d = rc.offset - ra.offset
                D = d if D is None else D
                if d != D:
                    return 0
        return D if D > 0 and D % 4 == 0 else 0

    # ------------------------------------------------------ gradient tables
    def _build_reduce_tables(self):
        flat = self.flat
        G = flat.G.data_ptr()
        segs = []  # (dst, src, count, part_stride, nparts)

        rb = 1 if self.bf16 else 0   # a bf16 Dense's kernel and bias gradients are bf16 values

        def dense_segs(spec: DenseSpec, wpart, bpart, splits):
            # (a split's partial may hold more input rows than the layer's:
            # a zero-padded input's gradient rows, which the sum skips)
            n = spec.fin * spec.w.ld
            segs.append((G + 4 * spec.w.offset, wpart.data_ptr(), n, wpart.stride(0), splits, rb))
            if spec.b is not None:
                segs.append((G + 4 * spec.b.offset, bpart.data_ptr(), spec.w.ld, spec.w.ld, splits, rb))

        paired = set()   # the paired towers' Dense segments (their group launch can finish them)
        first = set()    # the shared fp32 trunk's first Dense (its weight-gradient launch can finish it)
        for k, lb in enumerate(self.trunk + self.actor + self.critic):
            n0 = len(segs)
            dense_segs(lb.spec.dense, lb.wpart, lb.bpart, lb.splits)
            if self.chain_ln and k >= len(self.trunk):
                paired.update(range(n0, len(segs)))
            elif k == 0 and self.trunk:
                first.update(range(n0, len(segs)))
            if lb.spec.ln is not None:
                F = lb.spec.fout
                segs.append((G + 4 * lb.spec.ln["scale"].offset, lb.lnpart.data_ptr(), F, 2 * F, lb.lnblocks, 0))
                segs.append((G + 4 * lb.spec.ln["bias"].offset, lb.lnpart.data_ptr() + 4 * F, F, 2 * F,
                             lb.lnblocks, 0))
        p = self.prog
        if p.shared_head:
            dense_segs(p.head_a, self.HWPART, self.HBPART, self.head_splits)
        else:
            dense_segs(p.head_a, self.HAWPART, self.HABPART, self.ha_splits)
            dense_segs(p.head_c, self.HCWPART, self.HCBPART, self.hc_splits)
        if p.scale_region is not None:
            D = p.dist["dim"]
            segs.append((G + 4 * p.scale_region.offset, self.DSCALE.data_ptr(), D, D, self.loss_blocks, 0))
        segs += self._extra_segments(G)
        lib = _lib.load()
        assert lib.ppo_grad_reduce_segment_bytes() == 40 and lib.ppo_grad_reduce_chunk_bytes() == 16
        chunk = lib.ppo_grad_reduce_chunk_elems()
        few_parts, wide_parts = lib.ppo_grad_reduce_few_parts(), lib.ppo_grad_reduce_wide_parts()
        wide_chunk = lib.ppo_grad_reduce_wide_chunk_elems()
        dev = flat.device

        def pack(sel, slot0):
            """Device tables of the segments sel, their norm slots from slot0:
            (SEGS, CHUNKS, nchunks, nfew, nwide)."""
            sub = [segs[i] for i in sel]
            seg_bytes = b"".join(struct.pack("<QQqqii", d, s, c, st, n, f) for d, s, c, st, n, f in sub)
            # chunks of few-partial segments first (the kernel's wave-per-chunk
            # path); each keeps its slot in segment order, so the norm's fold
            # order does not depend on the split
            few, many, wide = [], [], []
            for i, (_, _, c, _, n, _) in enumerate(sub):
                dst = few if n <= few_parts else wide if n > wide_parts else many
                for start in range(0, c, wide_chunk if dst is wide else chunk):
                    slot = slot0 + len(few) + len(many) + len(wide)
                    dst.append(struct.pack("<iiq", i, slot, start))
            chunks = few + many + wide
            return (torch.tensor(list(seg_bytes) or [0], dtype=torch.uint8, device=dev),
                    torch.tensor(list(b"".join(chunks)) or [0], dtype=torch.uint8, device=dev),
                    len(chunks), len(few), len(wide))

        self.SEGS, self.CHUNKS, self.nchunks, self.nfew, self.nwide = pack(range(len(segs)), 0)
        self.SUMSQ = torch.zeros(self.nchunks, dtype=torch.float64, device=dev)
        self.SUMSQ1 = torch.zeros(1, dtype=torch.float64, device=dev)
        self.segments = segs
        # the paired towers' grouped weight-gradient launch finishing their
        # split-K sums itself (ppo_gemm_f32_dw_group_final): its tiles' norm
        # slots, then the other segments' chunks, reduced in the same launch
        self.dw_final = None
        shapes = self._pair_dw_shapes() if self.DW_FINAL and paired else None
        if shapes and all(sp in self.FINAL_SPLITS and (i >= 2 or -(-self.mb // sp) <= 512)
                          for i, (_, _, sp) in enumerate(shapes)):
            L = len(shapes)
            T = lib.ppo_gemm_f32_dw_final_slots(L, (ctypes.c_int * L)(*[m for m, _, _ in shapes]),
                                                (ctypes.c_int * L)(*[n for _, n, _ in shapes]))
            assert T > 0
            rest = [i for i in range(len(segs)) if i not in paired]
            SEGS, CHUNKS, nch, nfew, nwide = pack(rest, T)
            self.dw_final = {"T": T, "SEGS": SEGS, "CHUNKS": CHUNKS, "nchunks": nch, "nfew": nfew, "nwide": nwide,
                             "SUMSQ": torch.zeros(T + nch, dtype=torch.float64, device=dev),
                             "CNT": torch.zeros(9 * T, dtype=torch.int32, device=dev)}
        # the shared fp32 trunk's first layer: its weight gradient (the last
        # launch of a step, over the gathered observation rows) with the
        # gradient assembly of every leaf (ppo_gemm_f32_dw_group_final, one
        # problem; its own split-K sums in two levels at 32 or 64 splits)
        # (at the largest split count the launch sums that does not exceed the
        # layer's own: the GRU workload's 128 splits of 128 rows become 64)
        lb0 = self.trunk[0] if self.trunk else None
        sp0 = max([sp for sp in self.FINAL_SPLITS if lb0 is not None and sp <= lb0.splits] or [0])
        if (self.DW_FINAL and self.dw_final is None and sp0 > 0 and not self.bf16 and self.fused
                and self.prog.shared_head and lb0.spec.ln is None and -(-self.mb // sp0) <= 512
                and lb0.spec.dense.fin % 4 == 0 and lb0.spec.ld % 4 == 0):
            d = lb0.spec.dense
            T = lib.ppo_gemm_f32_dw_final_slots(1, (ctypes.c_int * 1)(d.fin), (ctypes.c_int * 1)(lb0.spec.ld))
            assert T > 0
            SEGS, CHUNKS, nch, nfew, nwide = pack([i for i in range(len(segs)) if i not in first], T)
            self.dw_final = {"T": T, "SEGS": SEGS, "CHUNKS": CHUNKS, "nchunks": nch, "nfew": nfew, "nwide": nwide,
                             "SUMSQ": torch.zeros(T + nch, dtype=torch.float64, device=dev),
                             "CNT": torch.zeros(9 * T, dtype=torch.int32, device=dev), "first": sp0}
        self._dw_finished = False

    # ------------------------------------------------------------- pieces
    def _normalize(self, st):
        """Advantage normalisation over the whole rollout (ppo.py:220-221)."""
        if self.cfg.normalize_advantage:
            self._call("ppo_normalize_advantages_f32", st, _p(self.ADV), self.B, _p(self.NORM_WS),
                       self.NORM_WS.numel())

    def _perm_size(self) -> int:
        """Items one epoch permutes: every sample (ppo.py:200)."""
        return self.B

    def _boot_rows(self) -> int:
        """Rows of the bootstrap forward: second.obs[-1] (ppo.py:208-212)."""
        return self.N

    def _dx_target(self, lb: LayerBufs):
        """(dst, epi, act, aux, ldaux) for the cotangent of layer lb's output."""
        s = lb.spec
        if s.ln is not None:
            return _p(lb.dY), EPI_STORE, 0, None, 0
        if s.act is None:
            return _p(lb.dZ), EPI_STORE, 0, None, 0
        aux = lb.PRE if s.act == "silu" else lb.Y
        return _p(lb.dZ), EPI_DACT, _act(s.act), _p(aux), s.ld

    def _plan_dw_group(self, layers, c):
        """Host argument arrays of ppo_gemm_bf16s_dw_group over a bf16 chain
        group's weight gradients: the first layer's from the observation copy
        (its gather indices set per call in ``rows[0]``), each later layer's
        from the previous layer's bf16 output, and with ``dhead16`` the shared
        head's from the top layer's bf16 output and the chain's bf16 head
        cotangents."""
        # (A, lda, B, ldb, C, ldc, M, N, splits, bias_grad) per problem
        probs = []
        for i, lb in enumerate(layers):
            s = lb.spec
            a, lda = (_p(self.OBS16), self.ldo16) if i == 0 else (_p(layers[i - 1].Y16), layers[i - 1].spec.ld)
            probs.append((a, lda, _p(lb.dZ16), s.ld, _p(lb.wpart), s.ld, s.dense.fin, s.ld, lb.splits, _p(lb.bpart)))
        if c.get("dhead16"):
            h, top = self.prog.head_a, layers[-1]
            d16, ld16 = c["dhead16"]
            probs.append((_p(top.Y16), top.spec.ld, d16, ld16, _p(self.HWPART), h.w.ld, h.fin, h.w.ld,
                          self.head_splits, _p(self.HBPART)))
        L = len(probs)
        vp = lambda xs: (ctypes.c_void_p * L)(*xs)
        i64 = lambda xs: (ctypes.c_int64 * L)(*xs)
        i32 = lambda xs: (ctypes.c_int * L)(*xs)
        col = lambda j: [p[j] for p in probs]
        g = {
            "A": vp(col(0)), "lda": i64(col(1)), "rows": vp([None] * L), "B": vp(col(2)), "ldb": i64(col(3)),
            "C": vp(col(4)), "ldc": i64(col(5)), "M": i32(col(6)), "N": i32(col(7)), "K": i32([self.mb] * L),
            "splits": i32(col(8)), "stride": i64([p[6] * p[5] for p in probs]), "bias_grad": vp(col(9)),
            "count": L,
        }
        order = ("A", "lda", "rows", "B", "ldb", "C", "ldc", "M", "N", "K", "splits", "stride", "bias_grad")
        g["args"] = [ctypes.addressof(g[k]) for k in order]
        return g

    def _bwd_layers(self, st, layers, x0, ldx0, idx0, side_dw=False):
        """Back-propagates through layers whose last output cotangent is in
        place; with side_dw (st the main stream) each later layer's fp32
        weight gradient runs on the side stream beside its input cotangent."""
        c = layers[0].chain16 if layers else None
        if c is not None and c["bwd"]:
            # every LayerNorm backward and input cotangent in one launch; then
            # the weight gradients from the bf16 cotangents it leaves
            top = layers[-1]
            h = self.prog.head_a
            hd = ((_p(self.DHEAD), h.w.ld, c["Whb"], h.w.ld, c["head_npad"]) if c.get("Whb")
                  else (None, 0, None, 0, 0))
            self._call("ppo_mlp16_ln_bwd", st, c["L"], _p(top.dY), top.spec.ld, self.mb, c["Wb"], c["Z"],
                       c["mean"], c["rstd"], c["g"], c["be"], c["dZ16"], top.spec.ld, c["part"], c["act"], *hd,
                       c["z16"], *c.get("dhead16", (None, 0)))
            if self.DW16_GROUP and len(layers) <= 8:
                g = c.get("dw_group")
                if g is None:
                    g = c["dw_group"] = self._plan_dw_group(layers, c)
                g["rows"][0] = idx0
                self._call("ppo_gemm_bf16s_dw_group", st, g["count"], *g["args"])
                return
            # the first layer's dW fills 198 of the 256 CUs: the later layers'
            # run beside it on the side stream
            s2 = self._fork(st) if self.DW16_SIDE else st
            for i in range(len(layers) - 1, -1, -1):
                lb = layers[i]
                s, d = lb.spec, lb.spec.dense
                if i == 0:
                    self._call("ppo_gemm_bf16s", st, A_COL, B_KN, 1, 1, _p(self.OBS16), self.ldo16, idx0,
                               _p(lb.dZ16), s.ld, _p(lb.wpart), s.ld, d.fin, s.ld, self.mb, lb.splits, d.fin * s.ld,
                               EPI_STORE, None, 0, 0, None, 0, _p(lb.bpart), self.DW16_TILE)
                else:
                    self._call("ppo_gemm_bf16s", s2, A_COL, B_KN, 1, 1, _p(layers[i - 1].Y16), layers[i - 1].spec.ld,
                               None, _p(lb.dZ16), s.ld, _p(lb.wpart), s.ld, d.fin, s.ld, self.mb, lb.splits,
                               d.fin * s.ld, EPI_STORE, None, 0, 0, None, 0, _p(lb.bpart), -1)
            self._join(st, s2)
            return
        for i in range(len(layers) - 1, -1, -1):
            lb = layers[i]
            s = lb.spec
            d = s.dense
            if i > 0:
                x, ldx, ridx = _p(layers[i - 1].Y), layers[i - 1].spec.ld, None
            else:
                x, ldx, ridx = x0, ldx0, idx0
            obs16 = i == 0 and self._reads_obs16(x, ridx, 0)
            y16 = i > 0 and layers[i - 1].Y16 is not None
            side_dw = st
            # bf16 cotangent of a LayerNorm layer: read by its dW and dX contractions
            dz16 = s.ln is not None and lb.dZ16 is not None and (obs16 or i > 0)
            if s.ln is not None:
                self._call("ppo_layernorm_act_bwd_bf16_out16" if dz16 else self._ln_bwd, st, _p(lb.dY), s.ld,
                           _p(lb.Z), s.ld, _p(lb.mean), _p(lb.rstd), self.flat.view(s.ln["scale"]),
                           self.flat.view(s.ln["bias"]), _p(lb.dZ16) if dz16 else _p(lb.dZ), s.ld, _p(lb.lnpart),
                           self.mb, s.fout, _act(s.act))
            dz = _p(lb.dZ16) if dz16 else _p(lb.dZ)
            if obs16:
                self._call("ppo_gemm_bf16s", st, A_COL, B_KN, 1, int(dz16), _p(self.OBS16), self.ldo16, ridx, dz,
                           s.ld, _p(lb.wpart), s.ld, d.fin, s.ld, self.mb, lb.splits, d.fin * s.ld, EPI_STORE, None,
                           0, 0, None, 0, _p(lb.bpart), self.DW16_TILE)
            elif y16 or dz16:
                a = _p(layers[i - 1].Y16) if y16 else x
                self._call("ppo_gemm_bf16s", st, A_COL, B_KN, int(y16), int(dz16), a, ldx, None, dz, s.ld,
                           _p(lb.wpart), s.ld, d.fin, s.ld, self.mb, lb.splits, d.fin * s.ld, EPI_STORE, None, 0, 0,
                           None, 0, _p(lb.bpart), -1)
            elif i == 0 and self._first_dw_final(st, layers, x, ldx, ridx):
                pass   # the first layer's weight gradient with every leaf's gradient assembly
            else:
                # a later layer's weight gradient runs on the side stream beside
                # its input cotangent (neither writes what the other reads)
                sd = self._fork(st) if i > 0 and side_dw and self.DW_SIDE else st
                self._gemm(sd, A_COL, B_KN, x, ldx, ridx, _p(lb.dZ), s.ld, _p(lb.wpart), s.ld, d.fin,
                          s.ld, self.mb, lb.splits, d.fin * s.ld, EPI_STORE, None, 0, None, None, 0, _p(lb.bpart),
                          -1)
                side_dw = sd
            if i > 0:
                dst, epi, act, aux, ldaux = self._dx_target(layers[i - 1])
                if dz16:
                    self._call("ppo_gemm_bf16s", st, A_ROW, B_NK, 1, 1, dz, s.ld, None, self._view16(d.w), d.w.ld,
                               dst, layers[i - 1].spec.ld, self.mb, d.fin, s.ld, 1, 0, epi, None, act, 1, aux,
                               ldaux, None, -1)
                else:
                    self._gemm(st, A_ROW, B_NK, _p(lb.dZ), s.ld, None, self.flat.view(d.w), d.w.ld,
                              dst, layers[i - 1].spec.ld, self.mb, d.fin, s.ld, 1, 0, epi, None, act, None, aux,
                              ldaux, None, -1)
            if side_dw != st:
                self._join(st, side_dw)

    def _fwd_boot_chain(self, st, x, ldx, nrows):
        """The critic tower's forward for the bootstrap rows in one launch."""
        c, boot = self._chain, self.boot_layers
        s0 = boot[0].spec
        self._call("ppo_mlp_ln_fwd_f32", st, 1, len(boot), x, ldx, None, nrows, s0.dense.fin, c["bW"],
                   s0.dense.w.ld, 256, c["bb"], c["bg"], c["bbe"], c["bZ"], c["bY"], s0.ld, c["bmean"], c["brstd"],
                   self._chain_eps, self._chain_act, 0, 0, 0, 0, None, 0)
        return _p(boot[-1].Y), boot[-1].spec.ld

    def _chain_fwd_args(self, x, ldx, rows_idx, nrows) -> tuple:
        """Arguments of ppo_mlp_ln_fwd_f32 after the stream for both towers'
        chains (which also write the kernels' transposed images for this
        step's backward)."""
        c, s0 = self._chain, self.actor[0].spec
        return (2, len(self.actor), x, ldx, rows_idx, nrows, s0.dense.fin, c["W"], s0.dense.w.ld, 256, c["b"], c["g"],
                c["be"], c["Z"], c["Y"], s0.ld, c["mean"], c["rstd"], self._chain_eps, self._chain_act, 0, self.pair,
                self._chain_rs, self._chain_ss, c["WT"], 256 * 256)

    def _fwd_pair(self, st, x, ldx, rows_idx, nrows):
        """Forward of the actor (tower 0) and critic (tower 1) towers, one
        launch per depth; both first layers read the same input rows."""
        D, sx = self.pair, 0
        if self.chain_ln:
            self._call("ppo_mlp_ln_fwd_f32", st, *self._chain_fwd_args(x, ldx, rows_idx, nrows))
            return
        for la, lc in zip(self.actor, self.critic):
            s = la.spec
            d = s.dense
            W = self.flat.view(d.w)
            Bb = self.flat.view(d.b) if d.b is not None else None
            if s.ln is not None:
                self._call("ppo_gemm_ln_act_fwd_f32_towers", st, 2, x, ldx, rows_idx, W, d.w.ld, Bb,
                           self.flat.view(s.ln["scale"]), self.flat.view(s.ln["bias"]), _p(la.Z), s.ld, _p(la.Y),
                           s.ld, _p(la.mean), _p(la.rstd), nrows, d.fin, s.fout, s.ln["eps"], _act(s.act), sx, D,
                           _tstride(la.Y, lc.Y), _tstride(la.mean, lc.mean))
            else:
                pre = _p(la.PRE) if la.PRE is not None else None
                self._call("ppo_gemm_f32_towers", st, 2, A_ROW, B_KN, x, ldx, rows_idx, W, d.w.ld, _p(la.Y), s.ld,
                           nrows, s.ld, d.fin, 1, 0, EPI_BIAS_ACT, Bb, _act(s.act), pre, None, 0, None, -1, sx, D,
                           _tstride(la.Y, lc.Y), D, _tstride(la.PRE, lc.PRE) if pre else 0, 0, 0)
            x, ldx, rows_idx, sx = _p(la.Y), s.ld, None, _tstride(la.Y, lc.Y)

    def _bwd_pair(self, st, x0, ldx0, idx0, chain_done=False):
        """Backward of the actor and critic towers, one launch per depth and
        contraction, once both last-layer output cotangents are in place
        (chain_done: the torso chains' backward already ran, in the forward's
        launch; only the weight gradients remain)."""
        D, A, C = self.pair, self.actor, self.critic
        if self.chain_ln:
            c = self._chain
            if not chain_done:
                self._call("ppo_mlp_ln_bwd_f32", st, 2, len(A), _p(A[-1].dY), A[-1].spec.ld, self.mb, c["Z"],
                           c["mean"], c["rstd"], c["g"], c["be"], c["WT"], 256, c["dZ"], A[0].spec.ld, c["part"],
                           self._chain_act, self._chain_rs, self._chain_ss, D, 256 * 256, self._chain_ps)
            g = self._pair_dw_group(x0, ldx0)
            if g is not None:
                # every weight gradient of both towers in one launch
                g["rows"][0] = g["rows"][1] = idx0
                if "final_args" in g:
                    # ... with their gradient assembly: the optimizer step reads them directly
                    self._call("ppo_gemm_f32_dw_group_final", st, g["count"], *g["final_args"])
                    self._dw_finished = True
                else:
                    self._call("ppo_gemm_f32_dw_group", st, g["count"], *g["args"])
                return
            for i, n, sx in self._dw_groups:
                la, lc = A[i], C[i]
                s = la.spec
                d = s.dense
                x, ldx, ridx = (x0, ldx0, idx0) if i == 0 else (_p(A[i - 1].Y), A[i - 1].spec.ld, None)
                fin = d.fin
                if i == 0 and self.obs_pad:
                    # the zero-padded observation copy, over its padded width
                    x, ldx, fin = _p(self.OBSP), self.obs_pad, self.obs_pad
                # problem k + 1 sits one (actor -> critic, or critic -> next actor) step after problem k
                self._call("ppo_gemm_f32_towers", st, n, A_COL, B_KN, x, ldx, ridx, _p(la.dZ), s.ld, _p(la.wpart),
                           s.ld, fin, s.ld, self.mb, la.splits, fin * s.ld, EPI_STORE, None, 0, None, None, 0,
                           _p(la.bpart), -1, sx, _tstride(la.dZ, lc.dZ), _tstride(la.wpart, lc.wpart), 0, 0, 0,
                           _tstride(la.bpart, lc.bpart))
            return
        for i in range(len(A) - 1, -1, -1):
            la, lc = A[i], C[i]
            s = la.spec
            d = s.dense
            if i > 0:
                x, ldx, ridx, sx = _p(A[i - 1].Y), A[i - 1].spec.ld, None, _tstride(A[i - 1].Y, C[i - 1].Y)
            else:
                x, ldx, ridx, sx = x0, ldx0, idx0, 0
            rs = _tstride(la.dZ, lc.dZ)
            if s.ln is not None and not self.chain_ln:
                self._call("ppo_layernorm_act_bwd_f32_towers", st, 2, _p(la.dY), s.ld, _p(la.Z), s.ld, _p(la.mean),
                           _p(la.rstd), self.flat.view(s.ln["scale"]), self.flat.view(s.ln["bias"]), _p(la.dZ),
                           s.ld, _p(la.lnpart), self.mb, s.fout, _act(s.act), rs, _tstride(la.mean, lc.mean), D,
                           _tstride(la.lnpart, lc.lnpart))
            self._call("ppo_gemm_f32_towers", st, 2, A_COL, B_KN, x, ldx, ridx, _p(la.dZ), s.ld, _p(la.wpart), s.ld,
                       d.fin, s.ld, self.mb, la.splits, d.fin * s.ld, EPI_STORE, None, 0, None, None, 0,
                       _p(la.bpart), -1, sx, rs, _tstride(la.wpart, lc.wpart), 0, 0, 0,
                       _tstride(la.bpart, lc.bpart))
            if i > 0 and not self.chain_ln:
                dst, epi, act, aux, ldaux = self._dx_target(A[i - 1])
                dst_c, _, _, aux_c, _ = self._dx_target(C[i - 1])
                self._call("ppo_gemm_f32_towers", st, 2, A_ROW, B_NK, _p(la.dZ), s.ld, None, self.flat.view(d.w),
                           d.w.ld, dst, A[i - 1].spec.ld, self.mb, d.fin, s.ld, 1, 0, epi, None, act, None, aux,
                           ldaux, None, -1, rs, D, _tstride(dst, dst_c), 0, 0,
                           _tstride(aux, aux_c) if aux is not None else 0, 0)

    def _head_back(self, st, layers, dhead, head: DenseSpec, wpart, bpart, splits, hx, ldhx, hidx):
        """Head dW and the cotangent of the head input."""
        top = layers[-1] if layers else None
        c = layers[0].chain16 if layers else None
        if c is not None and c.get("dhead16") and self.DW16_GROUP:
            pass  # the head's dW runs in the trunk's grouped dW launch, after the backward chain
        elif top is not None and top.Y16 is not None and hidx is None and head.w.ld % 4 == 0:
            # from the bf16 copy of the head input (the same bf16 values the
            # fp32 one rounds to, the same MFMA sequence and split boundaries)
            self._call("ppo_gemm_bf16s", st, A_COL, B_KN, 1, 0, _p(top.Y16), top.spec.ld, None, _p(dhead),
                       head.w.ld, _p(wpart), head.w.ld, head.fin, head.w.ld, self.mb, splits, head.fin * head.w.ld,
                       EPI_STORE, None, 0, 0, None, 0, _p(bpart), -1)
        else:
            self._gemm(st, A_COL, B_KN, hx, ldhx, hidx, _p(dhead), head.w.ld, _p(wpart), head.w.ld,
                      head.fin, head.w.ld, self.mb, splits, head.fin * head.w.ld, EPI_STORE, None, 0, None, None, 0,
                      _p(bpart), -1)
        if layers and not (c is not None and c.get("Whb")):  # else the backward chain takes it over
            dst, epi, act, aux, ldaux = self._dx_target(layers[-1])
            self._gemm(st, A_ROW, B_NK, _p(dhead), head.w.ld, None, self.flat.view(head.w),
                      head.w.ld, dst, layers[-1].spec.ld, self.mb, head.fin, head.w.ld, 1, 0, epi, None, act, None,
                      aux, ldaux, None, -1)

    # ----------------------------------------------------------- the update
    def bind(self, inputs: dict):
        """Pointers of the transition leaves (device tensors, time-major)."""
        self.inp = inputs

    def input_buffers(self) -> dict:
        """The executor's own rollout buffers (allocated on first use), which
        its captured update graphs read: obs [T + 1, N, obs] (first.obs =
        obs[:-1], second.obs = obs[1:]), action, reward, terminated,
        truncated, log_prob and value [T, N, ...]."""
        if getattr(self, "_own", None) is None:
            T, N, dev = self.T, self.N, self.flat.device
            f32 = dict(dtype=torch.float32, device=dev)
            b8 = dict(dtype=torch.bool, device=dev)
            dist = self.prog.dist
            own = {"obs": torch.zeros(T + 1, N, self.obs_dim, **f32),
                   "action": (torch.zeros(T, N, dtype=torch.int32, device=dev) if dist["kind"] == "categorical"
                              else torch.zeros(T, N, dist["dim"], **f32)),
                   "reward": torch.zeros(T, N, **f32), "terminated": torch.zeros(T, N, **b8),
                   "truncated": torch.zeros(T, N, **b8), "log_prob": torch.zeros(T, N, **f32),
                   "value": torch.zeros(T, N, **f32)}
            own.update(self._extra_input_buffers())
            self._own = own
            self.graphs: dict = {}
        return self._own

    def _extra_input_buffers(self) -> dict:
        return {}

    def issue(self, st: int, max_steps: int | None = None):
        """Enqueues one whole PPO.update on stream handle ``st``.  ``max_steps``
        stops after that many minibatch steps (the gradient buffer then holds
        the last step's gradient): a hook for parity tests."""
        inp, prog, cfg, chain = self.inp, self.prog, self.cfg, self.chain
        T, N, B, mb = self.T, self.N, self.B, self.mb
        obs, ldo = inp["obs"], self.obs_dim
        if self.obs_pad:
            self._call("ppo_pad_rows_f32", st, obs, ldo, _p(self.OBSP), self.obs_pad, B, ldo)
        if self.obs16:
            # bf16 copies the first-layer GEMMs read: the rollout's observations
            # (once per update) and the parameters (Adam refreshes the image)
            self._call("ppo_cast_bf16_2d", st, obs, ldo, _p(self.OBS16), self.ldo16, B, ldo)
            self._call("ppo_cast_bf16", st, _p(self.flat.P), _p(self.P16), self.flat.P.numel())
            self._pack16(st)
        # 1. bootstrap value of second.obs[-1] with the current parameters
        x, ldx, _ = inp["next_obs_last"], ldo, None
        if prog.shared_head:
            x, ldx, _ = self._fwd_layers(st, self.boot_layers, x, ldx, None, N)
            h = prog.head_a
            self._gemm(st, A_ROW, B_KN, x, ldx, None, self.flat.view(h.w), h.w.ld, _p(self.HEADB),
                      h.w.ld, N, h.w.ld, h.fin, 1, 0, EPI_BIAS_ACT, self.flat.view(h.b), 0, None, None, 0, None, -1)
            vcol = prog.head_out
        else:
            if self.chain_ln:
                x, ldx = self._fwd_boot_chain(st, x, ldx, N)
            else:
                x, ldx, _ = self._fwd_layers(st, self.boot_layers, x, ldx, None, N)
            h = prog.head_c
            self._gemm(st, A_ROW, B_KN, x, ldx, None, self.flat.view(h.w), h.w.ld, _p(self.HEADB),
                      h.w.ld, N, h.w.ld, h.fin, 1, 0, EPI_BIAS_ACT, self.flat.view(h.b), 0, None, None, 0, None, -1)
            vcol = 0
        self._call("ppo_act_fwd_f32", st, _p(self.HEADB) + 4 * vcol, self.HEADB.shape[1], _p(self.BOOT), 1, N, 1, 0)
        # 2. GAE
        self._call("ppo_gae_f32", st, inp["reward"], inp["terminated"], inp["truncated"], inp["value"],
                  _p(self.BOOT), None, None, _p(self.ADV), _p(self.RET), T, N, float(cfg.gamma),
                  float(cfg.gae_lambda), 0)
        self._normalize(st)
        self._pack_samples(st)
        # 3. epoch permutations of the flattened batch
        self._call("ppo_epoch_permutations", st, _p(self.KEY), self.E, B, _p(self.PERM), _p(self.PERM_WS),
                  self.PERM_WS.numel())
        # 4. minibatch steps
        dist = _lib.DIST[prog.dist["kind"]]
        A = prog.action_dim
        for e in range(self.E):
            for m in range(self.M):
                step = e * self.M + m
                if max_steps is not None and step >= max_steps:
                    self._finish_logs(st, step)
                    return
                idx = _p(self.PERM) + 4 * (e * B + m * mb)
                self._minibatch(st, idx, step, obs, ldo, dist, A)
                self._optimizer_step(st, step)
        self._finish_logs(st, self.E * self.M)
        self._call("ppo_count_advance", st, _p(self.flat.count), self.E * self.M, self._abort_word())

    def _abort_word(self):
        """Device int32 that, when nonzero, makes the optimizer steps and the
        count advance of this update write nothing (None: no such word)."""
        return None

    # Up to this many norm partials every Adam block folds itself (all 256
    # threads, about 16 loads each at most); above it one block folds them
    # first (a launch of its own).
    FOLD_NORM_MAX = 4096

    def _optimizer_step(self, st, step):
        """Gradient assembly (fixed-order sum of the split partials, with the
        squared-norm partials), then global-norm clip + Adam (ppo.py:182-191)."""
        chain = self.chain
        adam = chain.adam
        max_norm = chain.max_grad_norm if chain.max_grad_norm is not None else 0.0
        if self._dw_finished:
            # the weight-gradient launch assembled every gradient (tiles' norm slots, then the others')
            self._dw_finished = False
            fin = self.dw_final
            sumsq, nsq = fin["SUMSQ"], fin["T"] + fin["nchunks"]
        else:
            self._call("ppo_grad_reduce", st, _p(self.SEGS), _p(self.CHUNKS), self.nchunks, self.nfew, self.nwide,
                       _p(self.SUMSQ))
            sumsq, nsq = self.SUMSQ, self.nchunks
        if nsq <= self.FOLD_NORM_MAX:
            norm, nnorm = _p(sumsq), nsq
        else:
            self._call("ppo_sumsq_total", st, _p(sumsq), nsq, _p(self.SUMSQ1))
            norm, nnorm = _p(self.SUMSQ1), 1
        args = (_p(self.flat.P), _p(self.flat.G), _p(self.flat.MU), _p(self.flat.NU),
                _p(self.P16) if self.obs16 else None, self.flat.P.numel(), norm, nnorm, float(max_norm),
                adam.learning_rate, adam.b1, adam.b2, adam.eps, _p(self.flat.count), step, self._abort_word())
        if self.pair and self.fused and self._fwd_bwd_fused():
            tr = self.__dict__.get("_tr_args")
            if tr is None:
                offs, dsts = self._transposed_kernels()
                n = len(offs)
                tr = self._tr_args = (n, (ctypes.c_int64 * n)(*offs), (ctypes.c_void_p * n)(*dsts))
            self._call("ppo_adam_clip_wt_f32", st, *args, tr[0], ctypes.addressof(tr[1]), ctypes.addressof(tr[2]))
        else:
            self._call("ppo_adam_clip_f32", st, *args)
        if self.obs16:
            self._pack16(st)

    def _stats(self, step: int) -> int:
        """Loss-statistics partials of optimizer step ``step``."""
        return _p(self.STATS) + 8 * step * self.loss_blocks * self.nstat

    def _finish_logs(self, st, steps: int):
        """The logged scalars of the first ``steps`` optimizer steps (ppo.py:170-180)
        from their loss statistics, in one launch after the last step."""
        cfg = self.cfg
        self._call("ppo_loss_finalize_steps", st, _p(self.STATS), self.loss_blocks, self.mb, steps,
                   float(cfg.entropy_coefficient), float(cfg.value_coefficient), _p(self.LOGS))

    def _loss_adv(self) -> int:
        """Advantages the loss reads at the minibatch's sample indices."""
        return _p(self.ADV)

    def _ratio_out(self):
        """(pointer, envs, steps) where the fused loss keeps each row's ratio, or None."""
        return None

    def _head_a_io(self, la: LayerBufs):
        """(input, ld, cotangent destination, act, aux, ldaux) of head group a:
        the last layer's output, and where its cotangent goes."""
        da, epa, acta, auxa, ldauxa = self._dx_target(la)
        return _p(la.Y), la.spec.ld, da, (acta if epa == EPI_DACT else 0), auxa, ldauxa

    # the paired chains' forward and the fused heads + loss in one launch
    # (off: the chain launch, then the head loss launch)
    CHAIN_HEAD = True

    # after the first optimizer step of an update, the paired towers' forward
    # chain, heads + loss and backward chain run as one launch; each Adam step
    # writes the transposed kernels that launch's backward reads
    # (ppo_adam_clip_wt_f32), the first step's forward writes them itself
    FWD_BWD_FUSED = True

    def _fwd_bwd_fused(self) -> bool:
        return self.FWD_BWD_FUSED and self._chain_head and len(self.actor) > 1

    def _transposed_kernels(self):
        """(offsets in the flat parameters, transposed image pointers) of the
        paired towers' 256 x 256 kernels of layers 1.., actor then critic per
        layer: what ppo_adam_clip_wt_f32 keeps transposed for the fused
        forward + backward launch."""
        offs, dsts = [], []
        for l in range(1, len(self.actor)):
            for t, lb in enumerate((self.actor[l], self.critic[l])):
                offs.append(lb.spec.dense.w.offset)
                dsts.append(self.WT[l - 1, t].data_ptr())
        return offs, dsts

    @property
    def _chain_head(self) -> bool:
        v = self.__dict__.get("_chain_head_v")
        if v is None:
            v = self.__dict__["_chain_head_v"] = self._chain_head_fits()
        return v

    def _chain_head_fits(self) -> bool:
        """True when the paired towers' chain forward can run the fused heads
        + loss itself (ppo_mlp_ln_fwd_head_loss_f32): 256-wide chains feeding
        separate heads with no activation derivative, a minibatch whose head
        partials are kept per 16-row block, no per-row ratio output."""
        if not (self.CHAIN_HEAD and self.chain_ln and self.pair and not self.prog.shared_head):
            return False
        if self._ratio_out() is not None or self.actor[-1].spec.ld != 256 or self.prog.head_a.fin != 256:
            return False
        # the launch copies each head kernel into LDS from its 256-byte aligned
        # start (every leaf of the flat buffer is; a host-memory buffer, used
        # only to record launches, is checked by its leaf offsets)
        base = self.flat.P.data_ptr() if self.flat.P.is_cuda else 0
        if any((base + 4 * h.w.offset) % 256 for h in (self.prog.head_a, self.prog.head_c)):
            return False
        _, _, _, acta, _, _ = self._head_a_io(self.actor[-1])
        _, epc, _, _, _ = self._dx_target(self.critic[-1])
        return acta == 0 and epc != EPI_DACT and _lib.load().ppo_head_loss_blocks(self.mb) == -(-self.mb // 16)

    def _fused_head_loss(self, st, idx, step, dist, A, scale_ptr, act_i, act_f):
        args = self._head_loss_args(idx, step, dist, A, scale_ptr, act_i, act_f)
        ratio = self._ratio_out()
        if ratio is None:
            self._call("ppo_head_loss_f32", st, *args, self._sample_stride())
        else:
            self._call("ppo_head_loss_ratio_f32", st, *args, *ratio, self._sample_stride())

    # the fused loss reads log_prob, value, advantage, return and a
    # categorical action of each row from one 32-byte record per sample,
    # written once per update after the advantages are final: one 16-byte
    # load and one 64-byte sector per row instead of five scattered reads
    RECORDS = True

    def _sample_stride(self) -> int:
        return 8 if self.REC is not None else 1

    def _pack_samples(self, st):
        if self.REC is not None:
            act = self.inp["action"] if self.prog.dist["kind"] == "categorical" else None
            self._call("ppo_pack_samples", st, self.B, self.inp["log_prob"], self.inp["value"], self._loss_adv(),
                       _p(self.RET), act, _p(self.REC))

    def _head_loss_args(self, idx, step, dist, A, scale_ptr, act_i, act_f) -> tuple:
        """Arguments of ppo_head_loss_f32 after the stream, up to the sample
        stride (the per-sample inputs from the records when they are kept)."""
        prog, cfg, inp, mb = self.prog, self.cfg, self.inp, self.mb
        if prog.shared_head:
            la, lc = (self.trunk[-1] if self.trunk else None), None
            h = prog.head_a
            na = prog.head_out + 1
            wpa, bpa, wpc, bpc = self.HWPART, self.HBPART, None, None
        else:
            la, lc = self.actor[-1], self.critic[-1]
            h = prog.head_a
            na = prog.head_out
            wpa, bpa, wpc, bpc = self.HAWPART, self.HABPART, self.HCWPART, self.HCBPART
        ya, ldya, da, acta, auxa, ldauxa = self._head_a_io(la)
        if lc is not None:
            hc = prog.head_c
            dc, epc, actc, auxc, ldauxc = self._dx_target(lc)
            actc = actc if epc == EPI_DACT else 0
            c_args = (_p(lc.Y), lc.spec.ld, self.flat.view(hc.w), hc.w.ld, self.flat.view(hc.b))
            cd_args = (actc, auxc, ldauxc, dc, lc.spec.ld)
        else:
            c_args = (None, 0, None, 0, None)
            cd_args = (0, None, 0, None, 0)
        olp, vold, adv, ret = inp["log_prob"], inp["value"], self._loss_adv(), _p(self.RET)
        if self.REC is not None:
            rec = _p(self.REC)
            olp, vold, adv, ret = rec, rec + 4, rec + 8, rec + 12
            act_i = rec + 16 if act_i is not None else None
        return (dist, mb, idx, ya, ldya, self.flat.view(h.w), h.w.ld, self.flat.view(h.b), na, *c_args, h.fin, A,
                scale_ptr, act_i, act_f, olp, vold, adv, ret, acta, auxa,
                ldauxa, da, ldya, *cd_args, _p(wpa), _p(bpa), _p(wpc), _p(bpc), _p(self.DSCALE), self._stats(step),
                float(cfg.clip_coefficient), int(cfg.clip_value_loss), float(cfg.entropy_coefficient),
                float(cfg.value_coefficient), 1.0)

    def _minibatch(self, st, idx, step, obs, ldo, dist, A):
        prog, cfg, inp, mb = self.prog, self.cfg, self.inp, self.mb
        clip = float(cfg.clip_coefficient)
        scale_ptr = self.flat.view(prog.scale_region) if prog.scale_region is not None else None
        act_i = inp["action"] if dist == 0 else None
        act_f = inp["action"] if dist == 1 else None
        if self.fused:
            if prog.shared_head:
                self._fwd_layers(st, self.trunk, obs, ldo, idx, mb)
                self._fused_head_loss(st, idx, step, dist, A, scale_ptr, act_i, act_f)
                self._bwd_layers(st, self.trunk, obs, ldo, idx, side_dw=True)
            elif self.pair:
                if self._chain_head and self._fwd_bwd_fused() and step > 0:
                    # forward, heads + loss and the torso backward in one launch: the
                    # previous optimizer step wrote the transposed kernels it reads
                    c = self._chain
                    self._call("ppo_mlp_ln_fwd_head_loss_bwd_f32", st, *self._chain_fwd_args(obs, ldo, idx, mb),
                               *self._head_loss_args(idx, step, dist, A, scale_ptr, act_i, act_f),
                               self._sample_stride(), c["dZ"], c["part"], self._chain_ps)
                    self._bwd_pair(st, obs, ldo, idx, chain_done=True)
                    return
                if self._chain_head:
                    self._call("ppo_mlp_ln_fwd_head_loss_f32", st, *self._chain_fwd_args(obs, ldo, idx, mb),
                               *self._head_loss_args(idx, step, dist, A, scale_ptr, act_i, act_f),
                               self._sample_stride())
                else:
                    self._fwd_pair(st, obs, ldo, idx, mb)
                    self._fused_head_loss(st, idx, step, dist, A, scale_ptr, act_i, act_f)
                self._bwd_pair(st, obs, ldo, idx)
            else:
                s2 = self._fork(st)
                self._fwd_layers(st, self.actor, obs, ldo, idx, mb)
                self._fwd_layers(s2, self.critic, obs, ldo, idx, mb)
                self._join(st, s2)
                self._fused_head_loss(st, idx, step, dist, A, scale_ptr, act_i, act_f)
                s2 = self._fork(st)
                self._bwd_layers(st, self.actor, obs, ldo, idx)
                self._bwd_layers(s2, self.critic, obs, ldo, idx)
                self._join(st, s2)
            return
        if prog.shared_head:
            hx, ldhx, hidx = self._fwd_layers(st, self.trunk, obs, ldo, idx, mb)
            h = prog.head_a
            c = self.trunk[0].chain16 if self.trunk else None
            if c is None or not c.get("Wh"):  # else the trunk chain wrote the head outputs
                self._gemm(st, A_ROW, B_KN, hx, ldhx, hidx, self.flat.view(h.w), h.w.ld, _p(self.HEAD),
                          h.w.ld, mb, h.w.ld, h.fin, 1, 0, EPI_BIAS_ACT, self.flat.view(h.b), 0, None, None, 0,
                          None, -1)
            vcol = prog.head_out
            self._call("ppo_loss_f32", st, dist, mb, idx, _p(self.HEAD), h.w.ld, _p(self.HEAD) + 4 * vcol, h.w.ld,
                      A, scale_ptr, act_i, act_f, inp["log_prob"], inp["value"], _p(self.ADV), _p(self.RET),
                      _p(self.DHEAD), _p(self.DHEAD) + 4 * vcol, _p(self.DSCALE), self._stats(step), clip,
                      int(cfg.clip_value_loss), float(cfg.entropy_coefficient), float(cfg.value_coefficient), 1.0)
            self._head_back(st, self.trunk, self.DHEAD, h, self.HWPART, self.HBPART, self.head_splits, hx, ldhx,
                            hidx)
            self._bwd_layers(st, self.trunk, obs, ldo, idx, side_dw=True)
        else:
            ha, hc = prog.head_a, prog.head_c
            s2 = self._fork(st)
            ax, ldax, aidx = self._fwd_layers(st, self.actor, obs, ldo, idx, mb)
            cx, ldcx, cidx = self._fwd_layers(s2, self.critic, obs, ldo, idx, mb)
            self._gemm(st, A_ROW, B_KN, ax, ldax, aidx, self.flat.view(ha.w), ha.w.ld, _p(self.HA),
                      ha.w.ld, mb, ha.w.ld, ha.fin, 1, 0, EPI_BIAS_ACT, self.flat.view(ha.b), 0, None, None, 0,
                      None, -1)
            self._gemm(s2, A_ROW, B_KN, cx, ldcx, cidx, self.flat.view(hc.w), hc.w.ld, _p(self.HC),
                      hc.w.ld, mb, hc.w.ld, hc.fin, 1, 0, EPI_BIAS_ACT, self.flat.view(hc.b), 0, None, None, 0,
                      None, -1)
            self._join(st, s2)
            self._call("ppo_loss_f32", st, dist, mb, idx, _p(self.HA), ha.w.ld, _p(self.HC), hc.w.ld, A, scale_ptr,
                      act_i, act_f, inp["log_prob"], inp["value"], _p(self.ADV), _p(self.RET), _p(self.DHA),
                      _p(self.DHC), _p(self.DSCALE), self._stats(step), clip, int(cfg.clip_value_loss),
                      float(cfg.entropy_coefficient), float(cfg.value_coefficient), 1.0)
            s2 = self._fork(st)
            self._head_back(st, self.actor, self.DHA, ha, self.HAWPART, self.HABPART, self.ha_splits, ax, ldax,
                            aidx)
            self._head_back(s2, self.critic, self.DHC, hc, self.HCWPART, self.HCBPART, self.hc_splits, cx, ldcx,
                            cidx)
            self._bwd_layers(st, self.actor, obs, ldo, idx)
            self._bwd_layers(s2, self.critic, obs, ldo, idx)
            self._join(st, s2)

    # ------------------------------------------------------------ recording
    def record(self, max_steps: int | None = None) -> list:
        """The launch sequence of one update as (entry point, args) without
        running it (used by the benchmark to time single launches)."""
        calls = []
        self._call = lambda name, *args: calls.append((name, args))
        self._recording = True
        try:
            self.issue(0, max_steps=max_steps)
        finally:
            self._call = _lib.call
            self._recording = False
        return calls

    # ------------------------------------------------------ two towers at once
    def _fork(self, st: int) -> int:
        """Handle of the side stream, ordered after everything issued on st so
        far (inside a graph capture this forks the captured graph)."""
        if self._recording or self.side is None:
            return st
        side = self.side.cuda_stream
        if st == side:
            return st   # never a stream waiting on its own event
        self._call("ppo_stream_wait", side, st, self._ev_fork)
        return side

    def _join(self, st: int, st2: int):
        """Orders st after everything issued on the side stream st2."""
        if st2 == st:
            return
        self._call("ppo_stream_wait", st, st2, self._ev_join)
