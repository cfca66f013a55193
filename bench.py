"""Learner throughput of the PPO update on one MI355X.

A step is one complete PPO.update (bootstrap value, GAE, the epoch
permutations, and every minibatch forward/backward/loss/clip/Adam step) over
one synthetic rollout already resident in HBM.  The default workload is the
discrete Anakin configuration: obs [T=128, N=2048, 400] binary, 6 actions,
shared 2x256 ReLU torso, 4 epochs x 8 minibatches of 32768.

Prints one JSON line: learner samples/s, the roofline of the dominant kernel
(timed live with HIP events, launch by launch) and the oracle's CPU rate on a
bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
# the seeded synthetic rollouts (and the torch forward that fills their
# actions) are shared with the tests and live beside them
sys.path.insert(1, os.path.join(ROOT, "tests"))

PEAK = {"fp32_mfma": 157.3, "bf16_mfma": 2516.6, "hbm": 8000.0}  # TFLOP/s, TFLOP/s, GB/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--path", choices=("update", "step", "scan"), default="update",
                    help="update: the learner update (default); step: the rollout-side PPO.step "
                         "(forward + action sampling) for one rollout of T steps over N envs; scan: the "
                         "linear-recurrence scan forward + backward of an SSM torso")
    ap.add_argument("--scan-shape", default="1024,64,256", help="batch,steps,features of --path scan")
    ap.add_argument("--scan-dtype", choices=("f32", "bf16"), default="f32")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--launch-reps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline budget of the headline workload")
    ap.add_argument("--cpu-seconds-also", type=float, default=8.0, help="CPU baseline budget of each --also workload")
    ap.add_argument("--also", default="auto",
                    help="other workloads measured in the same run, into the line's 'configs' list: "
                         "'auto' (3,4,5,6 beside the default headline 2), 'none', or a comma list")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--detail", default=None, metavar="PATH",
                    help="also write the per-launch tables of every workload (JSON) to PATH")
    ap.add_argument("--profile-only", action="store_true", help="warmup + timed updates only")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (calibrates rocprofv3 FETCH/WRITE_SIZE)")
    return ap.parse_args()


def copy_probe(mib):
    """Five torch device-to-device copies of a known size: the reference
    dispatch against which the FETCH_SIZE / WRITE_SIZE counters are scaled."""
    import torch
    n = mib * (1 << 20) // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": 4 * n}), flush=True)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def measured_traffic(workload, kernel):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 --pmc
    summary (profiles/traffic.json), or None when that shape was not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(workload, {}).get(kernel)
    except (OSError, ValueError):
        return None
    if not rec:
        return None
    return 1024.0 * (rec["fetch_kib"] * rec["fetch_scale"] + rec["write_kib"] * rec["write_scale"])


def untower(name, args):
    """(entry point, arguments, towers) of a tower-batched launch as its
    single-tower entry point's call, and the number of towers it runs."""
    if not name.endswith("_towers"):
        return name, args, 1
    from boonta_amd import _lib
    base = name[: -len("_towers")]
    n = len(_lib.SIGNATURES[base][1])
    return base, (args[0],) + tuple(args[2:n + 1]), int(args[1])


def launch_work(name, args):
    """(flops, bytes) of one launch: algorithmic work of the call's shapes
    (GEMM: 2MNK FLOP; bandwidth-bound kernels: the bytes the computation must
    read and write once); a tower-batched launch does its towers' work."""
    name, args, towers = untower(name, args)
    flops, nbytes = _single_launch_work(name, args)
    return towers * flops, towers * nbytes


DW_GROUPS = ("ppo_gemm_bf16s_dw_group", "ppo_gemm_f32_dw_group", "ppo_gemm_f32_dw_group_final")


def dw_group_problems(args):
    """[(M, N, K, splits)] of a ppo_gemm_bf16s_dw_group or ppo_gemm_f32_dw_group
    call, read from its host argument arrays."""
    import ctypes
    L = int(args[1])
    ints = [list((ctypes.c_int * L).from_address(args[i])) for i in (9, 10, 11, 12)]
    return list(zip(*ints))


def gru_seq_shape(name, args):
    """(sequences, units, steps) of a GRU sequence launch."""
    i = {"ppo_gru_fwd_seq_f32": 23, "ppo_gru_fwd_seq_xw_f32": 20}.get(name, 22)   # after the stream: Bm, H, T
    return args[i], args[i + 1], args[i + 2]


def _single_launch_work(name, args):
    if name in DW_GROUPS:
        probs = dw_group_problems(args)
        e = 2.0 if name == "ppo_gemm_bf16s_dw_group" else 4.0   # operand element bytes
        if name == "ppo_gemm_f32_dw_group_final":
            # the operands and the finished gradient (its split partials are
            # the implementation's, not the algorithm's bytes)
            return (sum(2.0 * M * N * K for M, N, K, _ in probs),
                    sum(e * M * K + e * K * N + 4.0 * M * N for M, N, K, _ in probs))
        return (sum(2.0 * M * N * K for M, N, K, _ in probs),
                sum(e * M * K + e * K * N + 4.0 * M * N * S for M, N, K, S in probs))
    if name in ("ppo_gemm_f32", "ppo_gemm_bf16"):
        M, N, K = args[10], args[11], args[12]
        return 2.0 * M * N * K, 4.0 * (M * K + K * N + M * N)
    if name == "ppo_gemm_bf16s":
        M, N, K = args[12], args[13], args[14]
        ea, eb = (2.0 if args[3] else 4.0), (2.0 if args[4] else 4.0)
        return 2.0 * M * N * K, ea * M * K + eb * K * N + 4.0 * M * N * args[15]
    if name == "ppo_cast_bf16_2d":
        rows, cols, ldy = args[5], args[6], args[4]
        return 0.0, 4.0 * rows * cols + 2.0 * rows * ldy
    if name == "ppo_splits_bias_act_bf16":
        nsplit, rows, cols = args[4], args[9], args[10]
        return 0.0, 4.0 * rows * cols * (nsplit + 1)
    if name == "ppo_gemm_ln_act_fwd_f32":
        M, K, Fo = args[15], args[16], args[17]
        return 2.0 * M * Fo * K, 4.0 * (M * K + K * Fo + 2 * M * Fo)
    if name == "ppo_step_mlp_categorical_f32":
        rows, K0, L, ldwh = args[3], args[4], args[5], args[11]
        weights = K0 * 256 + (L - 1) * 256 * 256 + 256 * ldwh
        return 2.0 * rows * weights, 4.0 * (rows * K0 + weights + 3 * rows)
    if name == "ppo_sample_categorical_f32":
        rows, A = args[3], args[4]
        return 0.0, 4.0 * rows * (A + 4)
    if name == "ppo_sample_gaussian_f32":
        rows, D = args[5], args[6]
        return 0.0, 4.0 * rows * (3 * D + 3)
    if name == "ppo_gae_f32":
        T, N = args[10], args[11]
        return 0.0, 18.0 * T * N + 4.0 * N
    if name == "ppo_adam_clip_f32":
        n = args[6]
        return 0.0, 28.0 * n
    if name == "ppo_adam_clip_wt_f32":
        n, ntr = args[6], args[17]
        return 0.0, 28.0 * n + 4.0 * 256 * 256 * ntr
    if name == "ppo_head_loss_f32":
        rows, F, A = args[2], args[15], args[16]
        groups = 2 if args[10] else 1
        acts = (1 if args[26] else 0) + (1 if args[31] else 0)
        per_row = 4.0 * F * (2 * groups + acts) + 4.0 * 6 + (4.0 * A if args[1] == 1 else 0.0)
        return 0.0, rows * per_row
    if name == "ppo_mlp_ln_fwd_head_loss_f32":
        # the chain's work, then the fused heads + loss on its last outputs
        # (the entry point's arguments after the chain's are the head loss's)
        # (the heads read their inputs from the chain's last tiles in LDS: the
        # head loss's own reads of them are not counted)
        head = (args[0],) + tuple(args[27:])
        cf, cb = _single_launch_work("ppo_mlp_ln_fwd_f32", args[:27])
        hf, hb = _single_launch_work("ppo_head_loss_f32", head)
        rows, F, groups = head[2], head[15], (2 if head[10] else 1)
        return cf + hf, cb + hb - 4.0 * rows * F * groups
    if name == "ppo_mlp_ln_fwd_head_loss_bwd_f32":
        # the forward chain with the heads + loss, then the backward chain
        ff, fb = _single_launch_work("ppo_mlp_ln_fwd_head_loss_f32", args[:-3])
        towers, L, M = args[1], args[2], args[6]
        bf, bb = _single_launch_work("ppo_mlp_ln_bwd_f32", (args[0], towers, L, None, None, M))
        return ff + bf, fb + bb
    if name == "ppo_mlp_ln_fwd_f32":
        towers, L, M, K0 = args[1], args[2], args[6], args[7]
        weights = 256 * (K0 + 256 * (L - 1)) + 3 * 256 * L
        return towers * 2.0 * M * 256 * (K0 + 256 * (L - 1)), towers * 4.0 * (M * K0 + weights + M * L * (2 * 256 + 2))
    if name == "ppo_mlp_ln_bwd_f32":
        towers, L, M = args[1], args[2], args[5]
        weights = 256 * 256 * (L - 1) + 2 * 256 * L
        return towers * 2.0 * M * 256 * 256 * (L - 1), towers * 4.0 * (M * 256 + weights + M * L * (2 * 256 + 2))
    if name == "ppo_mlp16_ln_fwd":
        # split partials in; per layer Z (fp32, or bf16 with z16), Y16, mean, rstd out, the top layer's Y;
        # bf16 kernels; with the head, its outputs
        import ctypes
        L, nsplit, M = args[1], args[5], args[6]
        nh = args[21] if len(args) > 21 and args[19] else 0
        zb = 2.0 if len(args) > 24 and args[24] else 4.0
        ytab = ctypes.cast(args[12], ctypes.POINTER(ctypes.c_void_p)) if args[12] else None
        ys = sum(1 for l in range(L) if ytab is not None and ytab[l])  # layers whose fp32 output is written
        return (2.0 * M * 512 * (512 * (L - 1) + nh),
                4.0 * M * 512 * nsplit + 2.0 * 512 * (512 * (L - 1) + nh) + M * L * ((zb + 2.0) * 512 + 8)
                + 4.0 * M * 512 * ys + 4.0 * M * nh)
    if name == "ppo_pack_bf16_operand_padded":
        K, n_pad = args[3], args[5]
        return 0.0, 4.0 * K * n_pad
    if name == "ppo_mlp16_ln_bwd":
        # top cotangent (or the head's output cotangents) and per layer Z (fp32, or bf16 with z16), mean,
        # rstd in; dZ16 and the 32-row gradient sums out; bf16 kernels
        L, M = args[1], args[4]
        nh = args[18] if len(args) > 18 and args[17] else 0
        pad = (nh + 31) // 32 * 32
        zb = 2.0 if len(args) > 20 and args[20] else 4.0
        top = (4.0 * M * nh + 2.0 * 512 * pad) if nh else 4.0 * M * 512
        if len(args) > 22 and args[21]:  # the bf16 copy of the head cotangents
            top += 2.0 * M * args[22]
        return (2.0 * M * 512 * (512 * (L - 1) + pad),
                top + M * L * (zb * 512 + 8 + 2.0 * 512) + L * ((M + 31) // 32) * 4096.0
                + 2.0 * 512 * 512 * (L - 1))
    if name == "ppo_pack_bf16_operands":
        L, K, N = args[1], args[4], args[5]
        head = 8.0 * K * args[11] if len(args) > 11 and args[8] else 0.0
        return 0.0, 4.0 * L * K * N + head
    if name == "ppo_gru_fwd_seq_f32":
        Bm, H, T = gru_seq_shape(name, args)
        return 2.0 * Bm * H * 3 * H * T, 4.0 * T * Bm * (3 * H + H + H + 4 * H) + 4.0 * H * 3 * H
    if name == "ppo_gru_fwd_seq_xw_f32":
        # the input projections made in the launch: the GRU input rows read
        # instead of the projections, and their products
        Bm, H, T = gru_seq_shape(name, args)
        I = args[29]
        return (2.0 * Bm * H * 3 * H * T + 2.0 * T * Bm * I * 3 * H,
                4.0 * T * Bm * (I + H + H + 4 * H) + 4.0 * (H + I) * 3 * H)
    if name in ("ppo_gru_bwd_seq_f32", "ppo_gru_bwd_seq_dw_f32"):
        Bm, H, T = gru_seq_shape(name, args)
        flops = 2.0 * Bm * 3 * H * H * max(T - 1, 0)
        nbytes = 4.0 * T * Bm * (H + 4 * H + H + H + 4 * H) + 4.0 * H * 3 * H
        if name == "ppo_gru_bwd_seq_dw_f32":
            # the weight gradients: hp and e rows read, one partial per block of 16 sequences written
            I, parts = args[31], (Bm + 15) // 16
            flops += 2.0 * T * Bm * (H + I) * 3 * H
            nbytes += 4.0 * T * Bm * I + 4.0 * parts * (H + I + 2) * 3 * H
        return flops, nbytes
    if name in ("ppo_gru_fwd_step_f32",):
        Bm, H = args[-2], args[-1]
        return 2.0 * Bm * H * 3 * H, 4.0 * Bm * (3 * H + 2 * H + 6 * H) + 4.0 * H * 3 * H
    if name in ("ppo_gru_bwd_step_f32",):
        Bm, H = args[-2], args[-1]
        flops = 2.0 * Bm * 3 * H * H if args[1] else 0.0
        return flops, 4.0 * Bm * (3 * H + 2 * H + 7 * H) + (4.0 * H * 3 * H if args[1] else 0.0)
    if name in ("ppo_layernorm_act_fwd_f32", "ppo_layernorm_act_fwd_bf16"):
        rows, F = args[9], args[10]
        return 0.0, 4.0 * rows * (2 * F + 2)
    if name in ("ppo_layernorm_act_bwd_f32", "ppo_layernorm_act_bwd_bf16"):
        rows, F = args[12], args[13]
        return 0.0, 4.0 * rows * (3 * F + 2)
    if name == "ppo_layernorm_act_bwd_bf16_out16":
        rows, F = args[12], args[13]
        return 0.0, rows * (4.0 * 2 * F + 2.0 * F + 8.0)
    return 0.0, 0.0


def launch_shape(name, args):
    """[M, N, K] of a contraction launch (the one-launch step: [rows, 256,
    observation features, trunk layers]; a torso chain: [rows, 256, first
    layer's inputs, layers, towers]; a GRU sequence launch: [sequences,
    units, steps]; None for the others), with the tower count appended for a
    tower-batched launch."""
    base, bargs, towers = untower(name, args)
    shape = _single_launch_shape(base, bargs)
    return shape + [towers] if shape is not None and towers > 1 else shape


def _single_launch_shape(name, args):
    if name in DW_GROUPS:  # the first problem's [M, N, K] and the problem count
        M, N, K, _ = dw_group_problems(args)[0]
        return [M, N, K, int(args[1])]
    if name in ("ppo_gemm_f32", "ppo_gemm_bf16"):
        return list(args[10:13])
    if name == "ppo_gemm_bf16s":
        return list(args[12:15])
    if name == "ppo_gemm_ln_act_fwd_f32":
        return [args[15], args[17], args[16]]
    if name == "ppo_step_mlp_categorical_f32":
        return [args[3], 256, args[4], args[5]]
    if name in ("ppo_mlp_ln_fwd_f32", "ppo_mlp_ln_fwd_head_loss_f32", "ppo_mlp_ln_fwd_head_loss_bwd_f32"):
        return [args[6], 256, args[7], args[2], args[1]]
    if name == "ppo_mlp_ln_bwd_f32":
        return [args[5], 256, 256, args[2], args[1]]
    if name in ("ppo_gru_fwd_seq_f32", "ppo_gru_fwd_seq_xw_f32", "ppo_gru_bwd_seq_f32", "ppo_gru_bwd_seq_dw_f32"):
        return list(gru_seq_shape(name, args))
    if name == "ppo_mlp16_ln_fwd":
        return [args[6], 512, 512, args[1]]
    if name == "ppo_mlp16_ln_bwd":
        return [args[4], 512, 512, args[1]]
    if name.startswith("ppo_gru"):
        return [args[-2], args[-1]]
    return None


def launch_layout(name, args):
    name, args, _ = untower(name, args)
    if name in ("ppo_gemm_f32", "ppo_gemm_bf16", "ppo_gemm_bf16s"):
        return [args[1], args[2]]
    if name in DW_GROUPS:
        return [1, 0]
    return None


def launch_key(name, args):
    """Launches with the same entry point and shape do the same work."""
    base, bargs, towers = untower(name, args)
    if towers > 1 and base == "ppo_gemm_f32":
        return (towers,) + launch_key(base, bargs)
    if name in ("ppo_gemm_f32", "ppo_gemm_bf16"):
        return (name, args[1], args[2]) + tuple(args[10:16])
    if name == "ppo_gemm_bf16s":
        return (name,) + tuple(args[1:5]) + tuple(args[12:16])
    if name in DW_GROUPS:
        return (name,) + tuple(dw_group_problems(args))
    if name in ("ppo_gru_fwd_step_f32", "ppo_gru_bwd_step_f32"):
        return (name, args[-2], args[-1], bool(args[1]))
    if name in ("ppo_gru_fwd_seq_f32", "ppo_gru_fwd_seq_xw_f32", "ppo_gru_bwd_seq_f32", "ppo_gru_bwd_seq_dw_f32"):
        return (name,) + gru_seq_shape(name, args)
    if name == "ppo_mlp16_ln_fwd":
        return (name, args[1], args[5], args[6])
    if name == "ppo_mlp16_ln_bwd":
        return (name, args[1], args[4])
    return (name, id(args))


def time_launches(ex, reps, per_update_steps):
    """Per-launch durations of one update, each distinct launch of (bootstrap
    + GAE + permutations + one minibatch step) counted as many times as it
    occurs per update.

    ``ms_bracketed``: the launch inside a whole update issued eagerly on one
    stream, HIP events recorded between consecutive launches (so each launch
    runs with the caches its predecessors left), averaged over its
    occurrences; each interval also holds the launch's share of the gaps
    between eager launches.  ``ms_alone``: ``reps`` back-to-back repetitions
    of the launch on the same inputs (its inputs stay in the caches: an
    optimistic figure).  Returns (rows, launches per update)."""
    import torch
    from boonta_amd import _lib

    calls1 = ex.record(max_steps=1)
    stream = torch.cuda.current_stream()
    st = stream.cuda_stream
    # launches before the first minibatch step: those of an update stopped
    # before it, less its log finalize
    first_mb = len(ex.record(max_steps=0)) - 1
    full = ex.record()
    S = per_update_steps
    # the first step's launches, and those every later step repeats (the
    # first may differ: the Gaussian towers' first step writes the transposed
    # kernels its backward reads, later steps have them from Adam)
    step0 = calls1[first_mb:-1]
    step1 = ex.record(max_steps=2)[len(calls1) - 1:-1] if S > 1 else step0
    same = [n for n, _ in step0] == [n for n, _ in step1]
    later = [] if same else step1
    calls = calls1[:first_mb] + step0 + later + [calls1[-1]]
    counts = [1] * first_mb + [S if same else 1] * len(step0) + [S - 1] * len(later) + [1]
    if len(full) != first_mb + len(step0) + (S - 1) * len(step1) + 2:
        raise RuntimeError(f"unexpected launch count per update ({len(full)})")
    # position of each launch of the whole update in that template
    a0, a1 = first_mb, first_mb + (0 if same else len(step0))
    pos = (list(range(first_mb)) + [a0 + k for k in range(len(step0))]
           + [a1 + k % len(step1) for k in range((S - 1) * len(step1))] + [len(calls) - 1, None])
    if any(p is not None and full[k][0] != calls[p][0] for k, p in enumerate(pos)):
        raise RuntimeError("the minibatch steps of one update do not repeat one launch sequence")
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(full) + 1)]
    ev[0].record(stream)
    for k, (name, args) in enumerate(full):
        _lib.call(name, st, *args[1:])
        ev[k + 1].record(stream)
    ev[-1].synchronize()
    ctx_ms = [ev[k].elapsed_time(ev[k + 1]) for k in range(len(full))]
    rows, seen, by_pos = [], {}, {}
    for i, (name, args) in enumerate(calls):
        count = counts[i]
        key = launch_key(name, args)
        if key in seen:
            seen[key]["count"] += count
            by_pos[i] = seen[key]
            continue
        args = (st,) + tuple(args[1:])
        _lib.call(name, *args)  # warm
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            _lib.call(name, *args)
        e1.record(stream)
        e1.synchronize()
        flops, nbytes = launch_work(name, args)
        row = {"i": i, "name": name, "ms_alone": e0.elapsed_time(e1) / reps, "count": count, "flops": flops,
               "bytes": nbytes, "shape": launch_shape(name, args), "layout": launch_layout(name, args),
               "ctx": []}
        rows.append(row)
        seen[key] = row
        by_pos[i] = row
    for k, p in enumerate(pos):
        if p is not None:
            by_pos[p]["ctx"].append(ctx_ms[k])
    for r in rows:
        r["ms_bracketed"] = sum(r.pop("ctx")) / r["count"]
    return rows, len(full)


def in_update_durations(rows, launches: int, ms_per_update: float) -> float:
    """Sets each row's ``ms``: its bracketed interval less the mean per-launch
    excess of the bracketed eager update over the replayed graph's update,
    (sum of the intervals - ms_per_update) / launches, i.e. the time the
    launch takes inside the replayed update.  Returns that excess (ms)."""
    total = sum(r["ms_bracketed"] * r["count"] for r in rows)
    excess = max(0.0, (total - ms_per_update) / launches)
    for r in rows:
        r["ms"] = max(r["ms_bracketed"] - excess, 1e-6)
    return excess


def cpu_baseline(recipe, params, tr_dev, budget_s):
    """The oracle's update restatement in float32 numpy on the host
    (oracle.working_precision): the bootstrap forward, GAE over the whole
    rollout and the epoch permutations, then minibatch steps (gather of the
    minibatch rows from the host copy of the rollout, forward, backward,
    clip, Adam) until the time budget, extrapolated to E * M steps."""
    import oracle
    from boonta_amd.random import key as make_key
    from oracle import gae as ogae
    from oracle import nets as onets
    from oracle import ppo as oppo
    from oracle import prng as oprng

    f32 = np.float32
    plan = recipe.network.plan(recipe.obs_dim)
    T, N = recipe.T, recipe.N
    B, mb, E, M = recipe.batch, recipe.minibatch, recipe.cfg.update_epochs, recipe.cfg.num_minibatches
    cfg = {"clip_coefficient": recipe.cfg.clip_coefficient, "clip_value_loss": recipe.cfg.clip_value_loss,
           "entropy_coefficient": recipe.cfg.entropy_coefficient, "value_coefficient": recipe.cfg.value_coefficient}
    a = recipe.optimizer.adam
    opt = {"lr": a.learning_rate, "max_grad_norm": recipe.optimizer.max_grad_norm}
    # the rollout resident in host memory (copied before the clock starts)
    f, s = tr_dev.first, tr_dev.second
    host = lambda t: t.detach().cpu().numpy()
    obs, act, reward = host(f.obs), host(s.action), host(s.reward)
    term, trunc = host(s.terminated), host(s.truncated)
    logp, value, next_last = host(tr_dev.aux["log_prob"]), host(tr_dev.aux["value"]), host(s.obs[-1])
    if recipe.recurrent:
        first_done = host(f.terminated) | host(f.truncated)
        carry0, carry_last = host(tr_dev.carry[0]), host(tr_dev.carry[-1])
    key = make_key(recipe.seed)
    if recipe.algorithm == "pupo":
        return _cpu_baseline_pupo(recipe, params, plan, cfg, opt, key, budget_s, dict(
            obs=obs, first_done=first_done, action=act, reward=reward, terminated=term, truncated=trunc,
            log_prob=logp, value=value, carry0=carry0, carry_last=carry_last, next_obs_last=next_last,
            next_done_last=term[-1] | trunc[-1]))
    with oracle.working_precision(f32):
        p = oppo.tree_map(lambda x: np.asarray(x, f32), params)
        st = oppo.optimizer_init(p)
        t0 = time.perf_counter()
        if recipe.recurrent:
            seq_obs = np.stack([obs[-1], next_last], axis=1)
            seq_done = np.stack([first_done[-1], term[-1] | trunc[-1]], axis=1)
            boot = onets.recurrent_forward(p, plan, seq_obs, seq_done, carry_last)[1][:, -1]
        else:
            boot = onets.forward(p, plan, next_last)[1]
        adv, ret = ogae.gae(reward, term, trunc, value, boot, recipe.cfg.gamma, recipe.cfg.gae_lambda,
                            dtype=f32)
        perms = oprng.epoch_permutations(key, E, N if recipe.recurrent else B)
        t_pre = time.perf_counter() - t0
        steps, spent = 0, 0.0
        while spent < budget_s and steps < E * M:
            e, m = divmod(steps, M)
            t0 = time.perf_counter()
            if recipe.recurrent:
                # env-major sequence minibatches of N / M whole envs (recurrent_ppo.py:214-223)
                envs = perms[e].reshape(M, -1)[m]
                em = lambda x: np.moveaxis(np.take(x, envs, axis=1), 0, 1)
                _, _, grads = oppo.recurrent_loss_and_grad(p, plan, cfg, em(obs), em(first_done), carry0[envs],
                                                           em(act), em(logp), em(value), em(adv), em(ret))
            else:
                idx = perms[e].reshape(M, -1)[m]
                flat = lambda x: x.reshape((B,) + x.shape[2:])[idx]
                _, _, grads = oppo.loss_and_grad(p, plan, cfg, flat(obs), flat(act), flat(logp), flat(value),
                                                 flat(adv), flat(ret))
            p, st, _ = oppo.optimizer_update(grads, st, p, opt)
            spent += time.perf_counter() - t0
            steps += 1
    t_update = t_pre + E * M * spent / steps
    unit = f"{N // M} envs x {T} steps" if recipe.recurrent else f"{mb} rows"
    return {"value": B / t_update, "unit": "samples/s", "cores": _cores(), "kind": "port",
            "sample": f"float32 numpy oracle: bootstrap, GAE, {E} permutations ({t_pre:.2f} s) + {steps} of "
                      f"{E * M} minibatch steps of {unit} ({spent:.1f} s), extrapolated to one update"}


def _cores() -> int:
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    return min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))


def _cpu_baseline_pupo(recipe, params, plan, cfg, opt, key, budget_s, tr):
    """RecurrentPuPO's update restated by the oracle in float32: one step
    (bootstrap + first minibatch step, after one untimed warm-up run), then as
    many steps as the budget allows, the per-step time extrapolated to E * M
    steps."""
    import oracle
    from oracle import ppo as oppo

    E, M = recipe.cfg.update_epochs, recipe.cfg.num_minibatches
    c = recipe.cfg
    cfg = dict(cfg, gamma=c.gamma, gae_lambda=c.gae_lambda, update_epochs=E, num_minibatches=M,
               advantage_clip=c.advantage_clip, trace_clip=c.trace_clip, priority_exponent=c.priority_exponent,
               normalize_advantage=c.normalize_advantage)
    with oracle.working_precision(np.float32):
        p = oppo.tree_map(lambda x: np.asarray(x, np.float32), params)

        def run(k):
            t0 = time.perf_counter()
            oppo.recurrent_pupo_update(p, oppo.optimizer_init(p), plan, cfg, opt, tr, key, 0.2, max_steps=k)
            return time.perf_counter() - t0

        run(1)  # warm-up
        t1 = run(1)
        k = max(1, min(E * M, int(budget_s / max(t1, 1e-9))))
        per = (run(k) - t1) / (k - 1) if k > 1 else t1
    t_update = t1 + (E * M - 1) * per
    return {"value": recipe.batch / t_update, "unit": "samples/s", "cores": _cores(), "kind": "port",
            "sample": f"float32 numpy oracle of RecurrentPuPO.update: bootstrap + first step ({t1:.2f} s), "
                      f"{k} steps at {per:.2f} s each, extrapolated to {E * M} steps"}


BF16_KERNELS = ("ppo_gemm_bf16", "ppo_gemm_bf16s", "ppo_gemm_bf16s_dw_group", "ppo_mlp16_ln_fwd", "ppo_mlp16_ln_bwd")


def roofline_of(dom, total, workload):
    peak = PEAK["bf16_mfma"] if dom["name"] in BF16_KERNELS else PEAK["fp32_mfma"]
    # the roof the kernel meets first: its MFMA time at peak against its HBM time at peak
    if dom["flops"] > 0 and dom["flops"] / (peak * 1e12) >= dom["bytes"] / (PEAK["hbm"] * 1e9):
        achieved = dom["flops"] / (dom["ms"] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s",
                "frac": achieved / peak, "traffic": None}
    else:
        achieved = dom["bytes"] / (dom["ms"] * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": PEAK["hbm"], "unit": "GB/s",
                "frac": achieved / PEAK["hbm"], "traffic": None}
    roof["kernel"] = f"{dom['name']} layout={dom['layout']} MNK={dom['shape']}"
    roof["traffic"] = measured_traffic(workload, roof["kernel"])
    roof["avg_ms"] = dom["ms"]
    for k in ("ms_bracketed", "ms_alone"):
        if k in dom:
            roof["avg_" + k] = dom[k]
    roof["share_of_update"] = dom["ms"] * dom["count"] / total
    return roof


def launch_rows(rows):
    """Every timed launch with its own roofline: achieved TFLOP/s against the
    MFMA peak for contractions, achieved GB/s of algorithmic bytes against
    HBM for the rest (frac is null where no algorithmic work is modelled)."""
    out = []
    for r in rows:
        e = {k: r[k] for k in ("name", "layout", "shape", "ms", "ms_bracketed", "ms_alone", "count") if k in r}
        sec = r["ms"] * 1e-3
        peak = PEAK["bf16_mfma"] if r["name"] in BF16_KERNELS else PEAK["fp32_mfma"]
        # the roof a launch meets first: its MFMA time at peak against its HBM time at peak
        if r["flops"] > 0 and r["flops"] / (peak * 1e12) >= r["bytes"] / (PEAK["hbm"] * 1e9):
            e.update(bound="mfma", achieved=r["flops"] / sec / 1e12, frac=r["flops"] / sec / 1e12 / peak)
        elif r["bytes"] > 0:
            e.update(bound="hbm", achieved=r["bytes"] / sec / 1e9, frac=r["bytes"] / sec / 1e9 / PEAK["hbm"])
        else:
            e.update(bound=None, achieved=None, frac=None)
        out.append(e)
    return out


def _r(x, digits=4):
    """A float rounded to ``digits`` significant digits (None passes)."""
    return None if x is None else float(f"{x:.{digits}g}")


def short_kernel(label: str) -> str:
    """'name layout=[1, 0] MNK=[400, 256, 32768]' as 'name [1,0] [400,256,32768]'."""
    return label.replace("layout=", "").replace("MNK=", "").replace(", ", ",")


def compact_roofline(roof: dict) -> dict:
    """The headline's roofline object without the launch table's detail."""
    keep = {k: roof[k] for k in ("bound", "unit") if k in roof}
    keep["kernel"] = short_kernel(roof["kernel"])
    keep.update({k: _r(roof.get(k)) for k in ("achieved", "peak", "frac", "traffic", "avg_ms", "share_of_update")})
    return keep


def compact_config(m: dict) -> dict:
    """One extra workload as the headline line carries it."""
    out = {"workload": m["config"]["workload"], "value": _r(m["value"]), "ms_per_step": _r(m["ms_per_step"])}
    if "roofline" in m:
        out["frac"] = _r(m["roofline"]["frac"], 3)
        out["bound"] = m["roofline"]["bound"]
        out["kernel"] = short_kernel(m["roofline"]["kernel"])
    if "cpu_baseline" in m:
        out["cpu"] = _r(m["cpu_baseline"]["value"])
    return out


def emit(out: dict, args) -> None:
    """Prints the one-line JSON result on stdout (kept short: the per-launch
    tables go to stderr, and to --detail when given)."""
    detail = {"headline": out, "configs": out.pop("_configs_full", [])}
    line = dict(out)
    if "launches" in line:
        line.pop("launches")
        line.pop("launch_sum_ms", None)
        line.pop("launch_excess_ms", None)
    if "roofline" in line:
        line["roofline"] = compact_roofline(line["roofline"])
    for k in ("value", "ms_per_step"):
        line[k] = _r(line[k], 6)
    if "cpu_baseline" in line:
        line["cpu_baseline"] = dict(line["cpu_baseline"], value=_r(line["cpu_baseline"]["value"]))
    text = json.dumps(detail)
    log("detail " + text)
    if args.detail:
        with open(args.detail, "w") as f:
            f.write(text + "\n")
    print(json.dumps(line, separators=(",", ":")), flush=True)


def time_calls(calls, reps, count):
    """Each distinct launch of ``calls`` timed alone with HIP events on the
    launching stream (``reps`` back-to-back repetitions), counted ``count``
    times per measured unit."""
    import torch
    from boonta_amd import _lib

    stream = torch.cuda.current_stream()
    st = stream.cuda_stream
    rows = []
    for i, (name, args) in enumerate(calls):
        args = (st,) + tuple(args[1:])
        _lib.call(name, *args)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            _lib.call(name, *args)
        e1.record(stream)
        e1.synchronize()
        flops, nbytes = launch_work(name, args)
        row = {"i": i, "name": name, "ms": e0.elapsed_time(e1) / reps, "count": count, "flops": flops,
               "bytes": nbytes, "shape": launch_shape(name, args), "layout": launch_layout(name, args)}
        rows.append(row)
    return rows


def step_main(args, recipe, alg, state, params, dev):
    """Rollout-side PPO.step: one measured unit is the action selection of a
    whole rollout, T steps over N envs (forward + sample_and_log_prob per
    step, each step with its own key), captured once into a HIP graph and
    replayed with the observations resident in HBM."""
    import torch
    import synthetic
    from boonta_amd.random import key as make_key

    T, N, D = recipe.T, recipe.N, recipe.obs_dim
    roll = synthetic.rollout(recipe, T, N)
    obs_np = roll["obs"]
    obs = torch.from_numpy(obs_np).to(dev)
    ex = alg.step_executor(state, N, D)
    rec = recipe.recurrent
    if rec:
        # the carry entering every step, and each step's reset flags first.done[t]
        H = ex.prog.gru.H
        carries = torch.zeros(T + 1, N, H, dtype=torch.float32, device=dev)
        ft_np = np.concatenate([roll["first_done"][:1], roll["terminated"][:-1]], axis=0)
        ftr_np = np.concatenate([np.zeros((1, N), bool), roll["truncated"][:-1]], axis=0)
        ft, ftr = torch.from_numpy(ft_np).to(dev), torch.from_numpy(ftr_np).to(dev)
    dist = ex.prog.dist
    if dist["kind"] == "categorical":
        act = torch.zeros(T, N, dtype=torch.int32, device=dev)
    else:
        act = torch.zeros(T, N, dist["dim"], dtype=torch.float32, device=dev)
    lp = torch.zeros(T, N, dtype=torch.float32, device=dev)
    val = torch.zeros(T, N, dtype=torch.float32, device=dev)
    keys = torch.from_numpy(np.stack([make_key(5000 + t) for t in range(T)]).view(np.int32)).to(dev)

    def step_args(t):
        if rec:
            return (obs[t].data_ptr(), D, carries[t].data_ptr(), ft[t].data_ptr(), ftr[t].data_ptr(), 1.0,
                    carries[t + 1].data_ptr(), act[t].data_ptr(), lp[t].data_ptr(), val[t].data_ptr(),
                    keys[t].data_ptr())
        return (obs[t].data_ptr(), D, 1.0, act[t].data_ptr(), lp[t].data_ptr(), val[t].data_ptr(),
                keys[t].data_ptr())

    def issue_rollout():
        st = torch.cuda.current_stream().cuda_stream
        for t in range(T):
            ex.issue(st, *step_args(t))

    issue_rollout()
    torch.cuda.synchronize()
    g = None
    if not args.no_graph:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                issue_rollout()
        torch.cuda.current_stream().wait_stream(side)
    run = g.replay if g is not None else issue_rollout
    for w in range(args.warmup):
        run()
        torch.cuda.synchronize()
        log(f"warmup {w + 1}/{args.warmup} done")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    log(f"timed {args.steps} rollouts of action selection in {elapsed:.3f} s")
    if not torch.isfinite(lp).all() or not torch.isfinite(val).all():
        raise RuntimeError("non-finite step outputs")
    out = {
        "metric": "PPO.step action-selection samples/sec on 1 MI355X (rollout forward + sampling)",
        "value": T * N * args.steps / elapsed, "unit": "samples/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1000.0 * elapsed / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if ex.bf16 else "f32",
        "data": "synthetic (seeded observations of the workload's distribution, random-init network)",
        "config": {"workload": f"config {args.config}: {recipe.name} (PPO.step)", "T": T, "N": N, "obs": D,
                   "graph": not args.no_graph},
    }
    if not args.profile_only:
        calls = ex.record(*step_args(0))
        rows = time_calls(calls, args.launch_reps, T)
        total = sum(r["ms"] * r["count"] for r in rows)
        dom = max(rows, key=lambda r: r["ms"] * r["count"])
        out["roofline"] = roofline_of(dom, total, out["config"]["workload"])
        out["launches"] = launch_rows(rows)
        out["launch_sum_ms"] = total
        if not args.skip_cpu:
            log("cpu baseline ...")
            from oracle import nets as onets
            from oracle import sample as osample

            plan = recipe.network.plan(D)
            p64 = params
            spent, steps = 0.0, 0
            h = np.zeros((N, ex.prog.gru.H)) if rec else None
            while spent < args.cpu_seconds and steps < T:
                x = obs_np[steps]
                t1 = time.perf_counter()
                if rec:
                    done = (ft_np[steps] | ftr_np[steps])[:, None]
                    head, value, h, _ = onets.recurrent_forward(p64, plan, x[:, None, :], done, h)
                    head = head[:, 0]
                else:
                    head, value, _ = onets.forward(p64, plan, x)
                k = make_key(5000 + steps)
                if dist["kind"] == "categorical":
                    osample.categorical_sample(head, k, 1.0)
                elif dist.get("scale") is not None:
                    osample.gaussian_sample(head, np.asarray(onets.get(p64, dist["scale"])), k, 1.0)
                else:
                    Dm = dist["dim"]
                    osample.gaussian_sample(head[:, :Dm], head[:, Dm:], k, 1.0)
                spent += time.perf_counter() - t1
                steps += 1
            try:
                cores = len(os.sched_getaffinity(0))
            except AttributeError:
                cores = os.cpu_count()
            threads = int(os.environ.get("OMP_NUM_THREADS", cores))
            out["cpu_baseline"] = {"value": N * steps / spent, "unit": "samples/s", "cores": min(cores, threads),
                                   "kind": "port",
                                   "sample": f"oracle float64 numpy: {steps} steps of forward + sampling over "
                                             f"{N} envs ({spent:.1f} s)"}
    emit(out, args)


def scan_main(args):
    """Linear-recurrence scan (the SSM / MinGRU torso kernel): one step is a
    forward and a backward over [batch, steps, features] resident in HBM.
    Algorithmic bytes: forward reads a, b and writes h; backward reads a, h
    and the cotangent and writes da and db (init / dinit rows are extra)."""
    import torch
    from boonta_amd import _lib

    n, t, f = (int(x) for x in args.scan_shape.split(","))
    dt = torch.float32 if args.scan_dtype == "f32" else torch.bfloat16
    code = 0 if dt == torch.float32 else 1
    es = 4 if dt == torch.float32 else 2
    g = torch.Generator(device="cuda").manual_seed(0)
    a = (torch.rand((n, t, f), generator=g, device="cuda") * 0.9 + 0.05).to(dt)
    b = torch.rand((n, t, f), generator=g, device="cuda").to(dt)
    init = torch.randn((n, f), generator=g, device="cuda").to(dt)
    cot = torch.randn((n, t, f), generator=g, device="cuda").to(dt)
    h, da, db, dinit = torch.empty_like(a), torch.empty_like(a), torch.empty_like(a), torch.empty_like(init)
    st = torch.cuda.current_stream()
    fwd = ("ppo_linear_scan_fwd", (st.cuda_stream, code, a.data_ptr(), b.data_ptr(), init.data_ptr(),
                                   h.data_ptr(), n, t, f))
    bwd = ("ppo_linear_scan_bwd", (st.cuda_stream, code, a.data_ptr(), h.data_ptr(), init.data_ptr(),
                                   cot.data_ptr(), da.data_ptr(), db.data_ptr(), dinit.data_ptr(), n, t, f))

    def one():
        _lib.call(fwd[0], *fwd[1])
        _lib.call(bwd[0], *bwd[1])

    for _ in range(args.warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    per = {}
    for name, cargs in (fwd, bwd):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(args.launch_reps):
            _lib.call(name, *cargs)
        e1.record(st)
        e1.synchronize()
        per[name] = e0.elapsed_time(e1) / args.launch_reps
    elems = n * t * f
    nbytes = {"ppo_linear_scan_fwd": 3 * es * elems + es * n * f, "ppo_linear_scan_bwd": 5 * es * elems + 2 * es * n * f}
    dom = max(per, key=per.get)
    achieved = nbytes[dom] / (per[dom] * 1e-3) / 1e9
    out = {
        "metric": "linear-recurrence scan forward+backward elements/sec on 1 MI355X",
        "value": elems * args.steps / elapsed, "unit": "elements/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1000.0 * elapsed / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": args.scan_dtype, "data": "synthetic (uniform a, b)",
        "config": {"workload": f"linear scan [{n}, {t}, {f}] {args.scan_dtype}"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK["hbm"], "unit": "GB/s",
                     "frac": achieved / PEAK["hbm"], "traffic": None, "kernel": dom, "avg_ms": per[dom]},
        "launches": [{"name": k, "ms": v, "GB/s": nbytes[k] / (v * 1e-3) / 1e9} for k, v in per.items()],
    }
    if not args.skip_cpu:
        from oracle import scan as oscan
        k = max(1, min(n, 64))
        an, bn, inn, cn = (x[:k].float().cpu().numpy() for x in (a, b, init, cot))
        t1 = time.perf_counter()
        hh = oscan.forward(an, bn, inn)
        oscan.vjp(an, hh, inn, cn)
        spent = time.perf_counter() - t1
        out["cpu_baseline"] = {"value": k * t * f / spent, "unit": "elements/s", "cores": 1, "kind": "port",
                               "sample": f"oracle float64 numpy forward + VJP on {k} of the {n} sequences "
                                         f"({spent:.2f} s)"}
    emit(out, args)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the learner update runs on a "
              "single GPU; sharding it over several is a design, not built)", file=sys.stderr)
        sys.exit(2)
    import torch
    from boonta_amd import recipes

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.path == "scan":
        scan_main(args)
        return
    dev = torch.device("cuda:0")
    if args.path == "step":
        recipe = recipes.make(args.config)
        params = recipe.network.init(recipe.seed, recipe.obs_dim)["params"]
        alg = algorithm_of(recipe, not args.no_graph)
        state = alg.init_from_params({"params": params}, recipe.obs_dim)
        step_main(args, recipe, alg, state, params, dev)
        return
    out = {"metric": "PPO learner samples/sec on 1 MI355X + % of HBM/MFMA roofline per kernel",
           **measure_update(args, args.config, dev, headline=True)}
    extra = also_configs(args)
    if extra:
        full = [measure_update(args, c, dev, headline=False) for c in extra]
        out["configs"] = [compact_config(m) for m in full]
        out["_configs_full"] = full
    emit(out, args)


def algorithm_of(recipe, use_graph: bool):
    from boonta_amd.algorithms import PPO, RecurrentPPO, RecurrentPuPO
    cls = RecurrentPuPO if recipe.algorithm == "pupo" else RecurrentPPO if recipe.recurrent else PPO
    return cls(cfg=recipe.cfg, network=recipe.network, optimizer=recipe.optimizer, use_graph=use_graph)


def also_configs(args) -> list:
    """The other workloads measured in the same run (their lines go into
    ``configs``): by default the Gaussian, GRU, bf16 and RecurrentPuPO
    workloads beside the discrete Anakin headline, none for another headline or
    --profile-only."""
    if args.profile_only or args.also == "none":
        return []
    if args.also == "auto":
        return [3, 4, 5, 6] if args.config == 2 else []
    return [int(c) for c in args.also.split(",") if c and int(c) != args.config]


def measure_update(args, config: int, dev, headline: bool) -> dict:
    """One workload: seeded rollout resident in HBM, W untimed updates, K timed
    updates replayed from the HIP graph; then (unless --profile-only) each
    launch of one update timed alone for the per-kernel rooflines, and the
    CPU baseline."""
    import synthetic
    import torch
    from boonta_amd import recipes
    from boonta_amd.random import key as make_key

    recipe = recipes.make(config)
    log(f"workload {recipe.name}: T={recipe.T} N={recipe.N} obs={recipe.obs_dim} "
        f"{recipe.cfg.update_epochs}x{recipe.cfg.num_minibatches} minibatches of {recipe.minibatch}")
    params = recipe.network.init(recipe.seed, recipe.obs_dim)["params"]
    alg = algorithm_of(recipe, not args.no_graph)
    state = alg.init_from_params({"params": params}, recipe.obs_dim)
    # the rollout is written once into the learner's own input buffers (as an
    # Anakin rollout would be), so the timed updates read it in place
    tr = alg.rollout_buffers(state, recipe.T, recipe.N, recipe.obs_dim,
                             fill_from=synthetic.device_rollout(recipe, params, dev, recipe.seed))
    torch.cuda.synchronize()
    log("rollout ready")
    for w in range(args.warmup):
        alg.update(state, make_key(w), tr)
        torch.cuda.synchronize()
        log(f"warmup {w + 1}/{args.warmup} done")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        alg.update(state, make_key(100 + k), tr)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    log(f"timed {args.steps} updates in {elapsed:.3f} s")
    logs = alg.logs(state, recipe.T, recipe.N, recipe.obs_dim)
    if not all(np.isfinite(v).all() for v in logs.values()):
        raise RuntimeError("non-finite learner logs")
    out = {
        "value": recipe.batch * args.steps / elapsed, "unit": "samples/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1000.0 * elapsed / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if recipe.network.plan(recipe.obs_dim)["compute_dtype"] == "bfloat16" else "f32",
        "data": "synthetic seeded rollout, random-init network",
        "config": {"workload": f"config {config}: {recipe.name}", "T": recipe.T, "N": recipe.N,
                   "obs": recipe.obs_dim, "epochs": recipe.cfg.update_epochs,
                   "minibatches": recipe.cfg.num_minibatches, "minibatch": recipe.minibatch,
                   "global_batch": recipe.batch},
    }
    if not args.profile_only:
        ex = alg.executor(state, recipe.T, recipe.N, recipe.obs_dim)
        rows, launches = time_launches(ex, args.launch_reps, recipe.cfg.update_epochs * recipe.cfg.num_minibatches)
        out["launch_excess_ms"] = in_update_durations(rows, launches, out["ms_per_step"])
        total = sum(r["ms"] * r["count"] for r in rows)
        dom = max(rows, key=lambda r: r["ms"] * r["count"])
        out["roofline"] = roofline_of(dom, total, out["config"]["workload"])
        out["launches"] = launch_rows(rows)
        out["launch_sum_ms"] = total
        if not args.skip_cpu:
            log("cpu baseline ...")
            budget = args.cpu_seconds if headline else args.cpu_seconds_also
            out["cpu_baseline"] = cpu_baseline(recipe, params, tr, budget)
    del tr, alg, state
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    main()
