"""Host logic of the learner without a GPU: each workload's flat layout and its
full launch sequence, recorded instead of launched and checked against the C
signatures (arity, required pointers, buffer extents)."""
import numpy as np
import pytest
import ctypes
import struct

import torch

from boonta_amd import _lib, recipes
from boonta_amd.flat import load_tree, tree_from_flat, tree_to_numpy
from boonta_amd.learner import FlatState, MLPExecutor, Program
from boonta_amd.learner_rnn import RecurrentExecutor
from oracle import ppo as oppo

MLP_CONFIGS = [1, 2, 3]
FP32_CONFIGS = [1, 2, 3, 4]
ALL_CONFIGS = [1, 2, 3, 4, 5]


def small(config):
    r = recipes.make(config)
    if config == 2:
        return r.resized(T=16, N=64, num_minibatches=4, update_epochs=2)
    if config == 3:
        return r.resized(T=8, N=64, num_minibatches=4, update_epochs=2)
    if config == 4:
        return r.resized(T=8, N=64, num_minibatches=4, update_epochs=2)
    if config == 5:
        return r.resized(T=8, N=32, num_minibatches=2, update_epochs=2)
    return r


def executor(r, prog, flat, cls=None):
    if cls is None:
        cls = RecurrentExecutor if prog.gru is not None else MLPExecutor
    return cls(prog, flat, r.cfg, r.optimizer, r.T, r.N)


def fake_inputs(ex):
    return {k: 4096 * (i + 1) for i, k in enumerate(
        ["obs", "next_obs_last", "action", "reward", "terminated", "truncated", "log_prob", "value",
         "first_terminated", "first_truncated", "carry0", "carry_last"])}


@pytest.mark.parametrize("config", ALL_CONFIGS)
def test_recorded_launches_match_the_c_signatures(config):
    r = small(config)
    prog = Program(r.network.plan(r.obs_dim))
    flat = FlatState(prog, torch.device("cpu"))
    ex = executor(r, prog, flat)
    ex.bind(fake_inputs(ex))
    calls = ex.record()
    names = [n for n, _ in calls]
    steps = r.cfg.update_epochs * r.cfg.num_minibatches
    if prog.gru is not None:
        # two bootstrap steps, then T forward and T backward steps per minibatch
        assert names.count("ppo_gru_fwd_step_f32") == 2 + steps * r.T
        assert names.count("ppo_gru_bwd_step_f32") == steps * r.T
        assert names.count("ppo_sequence_rows") == 1
    # (the paired 256-wide towers' steps also keep their kernels transposed)
    adam = "ppo_adam_clip_wt_f32" if ex.pair and ex._fwd_bwd_fused() else "ppo_adam_clip_f32"
    assert names.count(adam) == steps and names.count("ppo_adam_clip_f32") + names.count("ppo_adam_clip_wt_f32") == steps
    assert names.count("ppo_loss_finalize_steps") == 1 and "ppo_loss_finalize" not in names
    # the norm's partials: the reduce's chunks, or, where the weight-gradient launch assembles the
    # gradients (the Gaussian towers' and the bf16 trunk's grouped launches), its tiles' and the rest's
    fin = ex.dw_final
    nsq = fin["T"] + fin["nchunks"] if fin is not None else ex.nchunks
    assert names.count("ppo_sumsq_total") == (0 if nsq <= ex.FOLD_NORM_MAX else steps)
    assert names.count("ppo_grad_reduce") == (0 if fin is not None else steps)
    if prog.bf16:
        # 43 actions: the unfused head GEMM + loss + head backward, every GEMM on bf16 MFMA
        assert names.count("ppo_loss_f32") == steps and "ppo_gemm_f32" not in names
        assert all(n != "ppo_layernorm_act_fwd_f32" for n in names)
    else:
        # every fp32 workload has torso features in front of its heads: the fused kernel runs (for
        # the Gaussian towers' chains, inside the forward chain's launch)
        # the Gaussian towers' chains, inside the forward chain's launch; after the first step
        # with the backward chain too)
        chained = names.count("ppo_mlp_ln_fwd_head_loss_f32") + names.count("ppo_mlp_ln_fwd_head_loss_bwd_f32")
        fused = names.count("ppo_head_loss_f32") + chained
        assert fused == steps and "ppo_loss_f32" not in names
        assert (chained == steps) == (config == 3)
    assert names[-1] == "ppo_count_advance"
    for name, args in calls:
        _, argtypes = _lib.SIGNATURES[name]
        assert len(args) == len(argtypes), (name, len(args), len(argtypes))
        if name in ("ppo_gemm_f32", "ppo_gemm_bf16"):
            (_, a_layout, b_layout, A, lda, rows, B, ldb, C, ldc, M, N, K, splits, stride, epi, bias, act, pre,
             aux, ldaux, bias_grad, tile) = args
            assert A and B and C and M > 0 and N > 0 and K > 0
            assert ldc >= N
            assert lda >= (K if a_layout == 0 else M)
            assert ldb >= (N if b_layout == 0 else K)
            if epi == 2:
                assert aux and ldaux >= N
            if splits > 1:
                assert stride >= M * ldc
        if name == "ppo_head_loss_f32":
            ha, wa, ba, dha, wpa, bpa, stats = args[4], args[6], args[8], args[27], args[34], args[35], args[39]
            assert all((ha, wa, ba, dha, wpa, bpa, stats))


@pytest.mark.parametrize("config", ALL_CONFIGS)
def test_flat_layout_round_trips_the_parameter_tree(config):
    r = recipes.make(config)
    prog = Program(r.network.plan(r.obs_dim))
    flat = FlatState(prog, torch.device("cpu"))
    params = r.network.init(3, r.obs_dim)["params"]
    load_tree(prog.layout, flat.P, params)
    back = tree_to_numpy(tree_from_flat(prog.layout, flat.P))
    a, b = dict(oppo.tree_leaves(params)), dict(oppo.tree_leaves(back))
    assert set(a) == set(b)
    for k in a:
        np.testing.assert_array_equal(np.asarray(a[k], np.float32), b[k])
    # every element outside the leaves is padding and stays zero
    used = np.zeros(prog.layout.size, bool)
    for lf in prog.layout.leaves.values():
        idx = lf.offset + sum(np.indices(lf.shape)[d] * lf.strides[d] for d in range(len(lf.shape)))
        assert not used[idx].any(), "leaves overlap"
        used[idx] = True
    assert np.all(flat.P.numpy()[~used] == 0)
    assert prog.layout.size % 64 == 0


def test_shared_heads_pack_logits_and_value_in_one_matrix():
    r = recipes.make(2)
    prog = Program(r.network.plan(r.obs_dim))
    assert prog.shared_head
    assert prog.head_a.w is prog.head_c.w
    assert prog.head_a.w.ld == 8            # 6 logits + 1 value, padded to 4
    lf_a = prog.layout.leaves[("head", "actor", "kernel")]
    lf_c = prog.layout.leaves[("head", "critic", "kernel")]
    assert lf_c.offset == lf_a.offset + 6 and lf_a.strides == (8, 1)


def test_unsupported_compositions_raise():
    from boonta_amd import networks as nn
    bad = nn.Network(feature_extractor=nn.FeatureExtractor(nn.Sequential([nn.Dense(8), nn.relu])),
                     head=nn.ActorCritic(actor=nn.Categorical(nn.Sequential([nn.Dense(8), nn.relu, nn.Dense(2)])),
                                         critic=nn.Dense(1)))
    with pytest.raises(NotImplementedError):
        Program(bad.plan(4))


@pytest.mark.parametrize("config", ALL_CONFIGS)
def test_rollout_step_launches_match_the_c_signatures(config):
    """PPO.step / RecurrentPPO.step (ppo.py:57-74, recurrent_ppo.py:71-96):
    the recorded launch sequence of one env step ends in the sampling launch
    and every call matches its C signature."""
    from boonta_amd.rollout import RecurrentStepExecutor, StepExecutor
    r = small(config)
    prog = Program(r.network.plan(r.obs_dim))
    flat = FlatState(prog, torch.device("cpu"))
    N = r.N
    if prog.gru is not None:
        ex = RecurrentStepExecutor(prog, flat, N)
        calls = ex.record(4096, r.obs_dim, 8192, 12288, 16384, 1.0, 20480, 24576, 28672, 32768)
        assert [n for n, _ in calls].count("ppo_gru_fwd_step_f32") == 1
    else:
        fused = StepExecutor(prog, flat, N)
        if fused.fused:
            # shared 256-wide fp32 trunk, categorical head: the whole step in one launch
            (name, args), = fused.record(4096, r.obs_dim, 1.0, 8192, 12288, 16384)
            assert name == "ppo_step_mlp_categorical_f32" and args[3] == N
            assert len(args) == len(_lib.SIGNATURES[name][1]) and args[5] == len(prog.trunk)
        ex = StepExecutor(prog, flat, N, fused=False)
        calls = ex.record(4096, r.obs_dim, 1.0, 8192, 12288, 16384)
    names = [n for n, _ in calls]
    want = "ppo_sample_categorical_f32" if prog.dist["kind"] == "categorical" else "ppo_sample_gaussian_f32"
    assert names[-1] == want and names.count(want) == 1
    for name, args in calls:
        _, argtypes = _lib.SIGNATURES[name]
        assert len(args) == len(argtypes), (name, len(args), len(argtypes))
    sample_args = calls[-1][1]
    assert sample_args[3 if want.endswith("categorical_f32") else 5] == N     # rows
    if config == 3:
        # 256-wide fp32 LayerNorm layers: Dense + LayerNorm + SiLU in one launch each
        assert names.count("ppo_gemm_ln_act_fwd_f32") == 8 and "ppo_layernorm_act_fwd_f32" not in names
    if prog.gru is None:
        assert fused.fused == (config == 2), "only the discrete Anakin network fits the one-launch step"


class PerLayerExecutor(MLPExecutor):
    """Paired towers issued layer by layer (the whole-chain launches off)."""
    CHAIN = False


class TowerDwExecutor(MLPExecutor):
    """Paired towers with the weight gradients as two tower-batched launches."""
    PAIR_DW_GROUP = False


def check_tower_dw_launches(r, prog, flat, steps):
    """The weight gradients as two ppo_gemm_f32_towers launches per step:
    layer 0 of both towers, then layers 1-3 of both towers."""
    ex = executor(r, prog, flat, cls=TowerDwExecutor)
    ex.bind(fake_inputs(ex))
    names = [n for n, _ in ex.record()]
    assert names.count("ppo_gemm_f32_towers") == 2 * steps and "ppo_gemm_f32_dw_group" not in names
    calls = ex.record(max_steps=1)
    dw = [a for n, a in calls if n == "ppo_gemm_f32_towers"]
    assert [a[1] for a in dw] == [2, 6]
    for a, first in zip(dw, (0, 1)):
        n, A_, B_, C_, bg = a[1], a[4], a[7], a[9], a[22]
        sa, sb, sc, sbg = a[24], a[25], a[26], a[30]
        for k in range(n):
            i, t = first + k // 2, k % 2
            lb = (ex.actor, ex.critic)[t][i]
            fin = lb.spec.dense.fin
            if i > 0:
                assert A_ + 4 * k * sa == (ex.actor, ex.critic)[t][i - 1].Y.data_ptr()
            else:
                # both towers read the observation rows: 87 features, so the
                # zero-padded copy over 88 columns (partials of 88 rows)
                assert sa == 0 and ex.obs_pad == 88 and A_ == ex.OBSP.data_ptr() and a[5] == 88
                fin = 88
                assert lb.wpart.shape[1] == 88
            assert B_ + 4 * k * sb == lb.dZ.data_ptr()
            assert C_ + 4 * k * sc == lb.wpart.data_ptr()
            assert bg + 4 * k * sbg == lb.bpart.data_ptr()
            assert a[11] == fin and a[13] == ex.mb and a[14] == lb.splits
            assert a[15] == fin * lb.spec.ld    # the partials' split stride


class NoFinalExecutor(MLPExecutor):
    """Paired towers whose grouped weight-gradient launch leaves the
    gradient assembly to the reduce launch."""
    DW_FINAL = False


def _segment_table(seg_tensor, n):
    """(dst, src, count, part_stride, nparts, flags) rows of a device segment table."""
    raw = bytes(seg_tensor.cpu().numpy().tobytes())
    return [struct.unpack_from("<QQqqii", raw, 40 * i) for i in range(n)]


def check_final_gradient_tables(ex, flat, args, adam_calls):
    """The finishing weight-gradient launch writes each paired Dense gradient
    (and bias) to its place in the flat gradient, reduces every other segment
    of the full table in the same launch, and the optimizer step folds its
    tile slots and chunk slots."""
    fin, g = ex.dw_final, ex._dwg
    G = flat.G.data_ptr()
    lbs = [lb for i in range(len(ex.actor)) for lb in (ex.actor[i], ex.critic[i])]
    assert list(args[15:19]) == [ctypes.addressof(g[k]) for k in ("G", "ldg", "g_rows", "Gb")]
    for k, lb in enumerate(lbs):
        d = lb.spec.dense
        assert g["G"][k] == G + 4 * d.w.offset and g["ldg"][k] == d.w.ld and g["g_rows"][k] == d.fin
        assert g["Gb"][k] == G + 4 * d.b.offset
    assert g["g_rows"][0] == 87 and g["M"][0] == 88     # the padded input's extra gradient row is dropped
    assert args[19] == fin["CNT"].data_ptr() and args[20] == fin["SUMSQ"].data_ptr()
    assert list(args[21:26]) == [fin["SEGS"].data_ptr(), fin["CHUNKS"].data_ptr(), fin["nchunks"], fin["nfew"],
                           fin["nwide"]]
    tiles = sum(-(-g["M"][k] // 64) * -(-g["N"][k] // 64) for k in range(g["count"]))
    assert fin["T"] == tiles and fin["CNT"].numel() == 9 * tiles and fin["SUMSQ"].numel() == tiles + fin["nchunks"]
    # the full table's segments = the finished Dense gradients + the rest table's
    full = _segment_table(ex.SEGS, len(ex.segments))
    nrest = len(ex.segments) - 2 * len(lbs)
    rest = _segment_table(fin["SEGS"], nrest)
    done = {g["G"][k] for k in range(len(lbs))} | {g["Gb"][k] for k in range(len(lbs))}
    assert sorted(rest + [r for r in full if r[0] in done]) == sorted(full)
    assert not any(r[0] in done for r in rest)
    # chunk slots of the rest start after the tiles'
    raw = bytes(fin["CHUNKS"].cpu().numpy().tobytes())
    slots = sorted(struct.unpack_from("<iiq", raw, 16 * i)[1] for i in range(fin["nchunks"]))
    assert slots == list(range(tiles, tiles + fin["nchunks"]))
    for a in adam_calls:
        assert a[7] == fin["SUMSQ"].data_ptr() and a[8] == tiles + fin["nchunks"]


class UnfusedChainExecutor(MLPExecutor):
    """Paired towers whose forward (with the heads + loss) and backward chains
    are separate launches at every step."""
    FWD_BWD_FUSED = False


def check_fused_forward_backward(ex, flat, calls):
    """The second step's fused launch: the first step's forward + head-loss
    arguments, with the transposed kernels as the backward's operand and the
    backward chain's own outputs; each Adam step keeps those kernels
    transposed (actor then critic per layer from layer 1)."""
    names = [n for n, _ in calls]
    first = [a for n, a in calls if n == "ppo_mlp_ln_fwd_head_loss_f32"]
    fused = [a for n, a in calls if n == "ppo_mlp_ln_fwd_head_loss_bwd_f32"]
    bwd = [a for n, a in calls if n == "ppo_mlp_ln_bwd_f32"]
    assert len(first) == len(fused) == len(bwd) == 1
    assert names.index("ppo_mlp_ln_fwd_head_loss_bwd_f32") > names.index("ppo_adam_clip_wt_f32")
    c = ex._chain
    f, u = fused[0], first[0]
    assert len(f) == len(u) + 3
    # same chain and head arguments except the step's gather indices and statistics
    same = [k for k in range(len(u)) if k not in (5, 29, 65)]
    assert [f[k] for k in same] == [u[k] for k in same]
    assert f[25] == c["WT"] and f[26] == 256 * 256
    assert list(f[-3:]) == [c["dZ"], c["part"], ex._chain_ps]
    # the backward reads the heads' input cotangents: dha and dhc = dha + stride_rows
    b = bwd[0]
    assert f[53] == b[3] and f[58] - f[53] == 4 * ex._chain_rs and f[54] == f[59] == b[4]
    for a in [a for n, a in calls if n == "ppo_adam_clip_wt_f32"]:
        n, offs, dsts = a[17], a[18], a[19]
        L = len(ex.actor)
        assert n == 2 * (L - 1)
        got_o = list((ctypes.c_int64 * n).from_address(offs))
        got_d = list((ctypes.c_void_p * n).from_address(dsts))
        want = [(lb.spec.dense.w.offset, ex.WT[l - 1, t].data_ptr())
                for l in range(1, L) for t, lb in enumerate((ex.actor[l], ex.critic[l]))]
        assert list(zip(got_o, got_d)) == want


def test_gaussian_update_without_the_fused_chains_runs_them_per_step():
    r = small(3)
    prog = Program(r.network.plan(r.obs_dim))
    flat = FlatState(prog, torch.device("cpu"))
    ex = executor(r, prog, flat, cls=UnfusedChainExecutor)
    ex.bind(fake_inputs(ex))
    names = [n for n, _ in ex.record()]
    steps = r.cfg.update_epochs * r.cfg.num_minibatches
    assert names.count("ppo_mlp_ln_fwd_head_loss_f32") == steps and names.count("ppo_mlp_ln_bwd_f32") == steps
    assert "ppo_mlp_ln_fwd_head_loss_bwd_f32" not in names and "ppo_adam_clip_wt_f32" not in names
    assert names.count("ppo_adam_clip_f32") == steps


def test_gaussian_update_without_the_finishing_launch_reduces_its_gradients():
    r = small(3)
    prog = Program(r.network.plan(r.obs_dim))
    flat = FlatState(prog, torch.device("cpu"))
    ex = executor(r, prog, flat, cls=NoFinalExecutor)
    ex.bind(fake_inputs(ex))
    names = [n for n, _ in ex.record()]
    steps = r.cfg.update_epochs * r.cfg.num_minibatches
    assert ex.dw_final is None and "ppo_gemm_f32_dw_group_final" not in names
    assert names.count("ppo_gemm_f32_dw_group") == steps and names.count("ppo_grad_reduce") == steps
    adam = [a for n, a in ex.record(max_steps=1) if n in ("ppo_adam_clip_f32", "ppo_adam_clip_wt_f32")]
    assert adam[0][7] == ex.SUMSQ.data_ptr() and adam[0][8] == ex.nchunks


def test_gaussian_update_runs_each_torso_chain_in_one_launch():
    r = small(3)
    prog = Program(r.network.plan(r.obs_dim))
    flat = FlatState(prog, torch.device("cpu"))
    ex = executor(r, prog, flat)
    ex.bind(fake_inputs(ex))
    assert ex.chain_ln
    names = [n for n, _ in ex.record()]
    steps = r.cfg.update_epochs * r.cfg.num_minibatches
    # per minibatch step: the forward chain of both towers (which also writes
    # the kernels' transposed images) with the fused heads + loss in the same
    # launch, the backward chain and every weight gradient of both towers in
    # one launch; the critic's bootstrap chain once
    calls = ex.record(max_steps=1)
    # (from the second step on, the backward chain runs in the forward's launch)
    assert names.count("ppo_mlp_ln_fwd_head_loss_f32") == 1 and "ppo_head_loss_f32" not in names
    assert names.count("ppo_mlp_ln_fwd_head_loss_bwd_f32") == steps - 1
    assert names.count("ppo_mlp_ln_fwd_f32") == 1
    assert names.count("ppo_mlp_ln_bwd_f32") == 1
    # ... which also assembles the gradients: no reduce launch per step
    assert names.count("ppo_gemm_f32_dw_group_final") == steps and "ppo_gemm_f32_towers" not in names
    assert "ppo_gemm_f32_dw_group" not in names and "ppo_grad_reduce" not in names
    assert names.count("ppo_pad_rows_f32") == 1   # the padded observation copy, once per update
    dwg = [a for n, a in calls if n == "ppo_gemm_f32_dw_group_final"]
    assert len(dwg) == 1 and dwg[0][1] == 2 * len(ex.actor)
    adam = [a for n, a in calls if n == "ppo_adam_clip_wt_f32"]
    assert len(adam) == 1
    check_final_gradient_tables(ex, flat, dwg[0], adam)
    g = ex._dwg
    fwd = [a for n, a in calls if n == "ppo_mlp_ln_fwd_head_loss_f32"][0]
    idx = fwd[5]   # the step's gather indices
    # the heads read the last layer of both towers; their input cotangents are the backward chain's dY
    c0 = 27   # first head-loss argument
    la, lc = ex.actor[-1], ex.critic[-1]
    assert fwd[c0 + 2] == idx and fwd[c0 + 3] == la.Y.data_ptr() and fwd[c0 + 9] == lc.Y.data_ptr()
    assert fwd[c0 + 26] == la.dY.data_ptr() and fwd[c0 + 31] == lc.dY.data_ptr()
    for k in range(g["count"]):
        i, t = k // 2, k % 2
        lb = (ex.actor, ex.critic)[t][i]
        if i > 0:
            prev = (ex.actor, ex.critic)[t][i - 1]
            assert g["A"][k] == prev.Y.data_ptr() and g["lda"][k] == prev.spec.ld and g["rows"][k] is None
            assert g["M"][k] == lb.spec.dense.fin
        else:
            # the zero-padded observation copy (87 -> 88 columns), gathered
            assert g["A"][k] == ex.OBSP.data_ptr() and g["lda"][k] == 88 and g["M"][k] == 88
            assert g["rows"][k] == idx and lb.wpart.shape[1] == 88
        assert g["B"][k] == lb.dZ.data_ptr() and g["C"][k] == lb.wpart.data_ptr()
        assert g["bias_grad"][k] == lb.bpart.data_ptr() and g["splits"][k] == lb.splits
        assert g["K"][k] == ex.mb and g["N"][k] == lb.spec.ld and g["stride"][k] == g["M"][k] * lb.spec.ld
    check_tower_dw_launches(r, prog, flat, steps)
    assert names.count("ppo_gemm_f32") == 1   # the bootstrap value head
    for gone in ("ppo_gemm_ln_act_fwd_f32", "ppo_gemm_ln_act_fwd_f32_towers", "ppo_layernorm_act_fwd_f32",
                 "ppo_layernorm_act_bwd_f32", "ppo_layernorm_act_bwd_f32_towers", "ppo_stream_wait"):
        assert gone not in names, gone
    # every table entry is the actor's pointer, and it plus the tower stride
    # is the critic's pointer of the same layer
    T = ex._chain_keep
    D = ex.pair
    for l, (a, c) in enumerate(zip(ex.actor, ex.critic)):
        s = a.spec
        assert T["W"][l] == flat.view(s.dense.w) and T["W"][l] + 4 * D == flat.view(c.spec.dense.w)
        assert T["g"][l] + 4 * D == flat.view(c.spec.ln["scale"])
        assert T["be"][l] + 4 * D == flat.view(c.spec.ln["bias"])
        assert T["b"][l] + 4 * D == flat.view(c.spec.dense.b)
        for key, attr, stride in (("Z", "Z", ex._chain_rs), ("Y", "Y", ex._chain_rs), ("dZ", "dZ", ex._chain_rs),
                                  ("mean", "mean", ex._chain_ss), ("rstd", "rstd", ex._chain_ss),
                                  ("part", "lnpart", ex._chain_ps)):
            assert T[key][l] == getattr(a, attr).data_ptr(), key
            assert T[key][l] + 4 * stride == getattr(c, attr).data_ptr(), key
        assert a.lnpart.shape[0] == _lib.load().ppo_mlp_ln_bwd_blocks(ex.mb)
    # the forward writes each tower's kernel of layers 1.. transposed into WT[layer - 1, tower]
    for l in range(1, len(ex.actor)):
        assert T["WT"][l] == ex.WT[l - 1, 0].data_ptr()
    fwd = [a[:27] for n_, a in calls if n_ in ("ppo_mlp_ln_fwd_f32", "ppo_mlp_ln_fwd_head_loss_f32")]
    assert [a[-2] for a in fwd] == [None, ex._chain["WT"]]   # the bootstrap chain writes none
    assert fwd[1][-1] == ex.WT[0, 1].data_ptr() - ex.WT[0, 0].data_ptr() >> 2
    # the bootstrap chain runs the critic's own layers
    for l, lb in enumerate(ex.boot_layers):
        assert T["bW"][l] == flat.view(ex.critic[l].spec.dense.w) and T["bY"][l] == lb.Y.data_ptr()
    check_fused_forward_backward(ex, flat, ex.record(max_steps=2))


def test_gaussian_update_pairs_its_towers_layer_by_layer():
    r = small(3)
    prog = Program(r.network.plan(r.obs_dim))
    flat = FlatState(prog, torch.device("cpu"))
    ex = PerLayerExecutor(prog, flat, r.cfg, r.optimizer, r.T, r.N)
    ex.bind(fake_inputs(ex))
    assert not ex.chain_ln
    calls = ex.record()
    names = [n for n, _ in calls]
    steps = r.cfg.update_epochs * r.cfg.num_minibatches
    # the actor and critic towers share every launch of a minibatch step: 4
    # Dense + LayerNorm + SiLU forwards, 4 LayerNorm backwards, 4 dW and 3
    # input-cotangent contractions; the critic's bootstrap forward runs alone
    assert ex.pair == prog.critic_layers[0].dense.w.offset - prog.actor_layers[0].dense.w.offset
    assert names.count("ppo_gemm_ln_act_fwd_f32_towers") == 4 * steps
    assert names.count("ppo_gemm_ln_act_fwd_f32") == 4
    assert names.count("ppo_layernorm_act_bwd_f32_towers") == 4 * steps
    assert names.count("ppo_gemm_f32_towers") == 7 * steps
    assert names.count("ppo_gemm_f32") == 1   # the bootstrap value head
    assert "ppo_layernorm_act_fwd_f32" not in names and "ppo_layernorm_act_bwd_f32" not in names
    assert "ppo_stream_wait" not in names

    # every tower-1 operand is tower 0's pointer plus its stride, and lands on
    # the critic's own buffer or parameter region of the same depth
    def ranges(layers):
        out = []
        for lb in layers:
            for t in (lb.Y, lb.Z, lb.PRE, lb.mean, lb.rstd, lb.dY, lb.dZ, lb.wpart, lb.bpart, lb.lnpart):
                if t is not None:
                    out.append((t.data_ptr(), t.data_ptr() + 4 * t.numel()))
        return out

    def regions(layers):
        out = set()
        for s in layers:
            out.add(flat.view(s.dense.w))
            if s.dense.b is not None:
                out.add(flat.view(s.dense.b))
            if s.ln is not None:
                out |= {flat.view(s.ln["scale"]), flat.view(s.ln["bias"])}
        return out

    actor_bufs, critic_bufs = ranges(ex.actor), ranges(ex.critic)
    actor_params, critic_params = regions(prog.actor_layers), regions(prog.critic_layers)
    inside = lambda x, rs: any(a <= x < b for a, b in rs)
    checked = 0
    for name, args in calls:
        if name == "ppo_gemm_ln_act_fwd_f32_towers":
            sx, sp, sr, ss = args[-4:]
            params = [(args[5], sp), (args[7], sp), (args[8], sp), (args[9], sp)]
            bufs = [(args[10], sr), (args[12], sr), (args[14], ss), (args[15], ss)] + ([(args[2], sx)] if sx else [])
        elif name == "ppo_layernorm_act_bwd_f32_towers":
            sr, ss, sp, spart = args[-4:]
            params = [(args[8], sp), (args[9], sp)]
            bufs = [(args[2], sr), (args[4], sr), (args[6], ss), (args[7], ss), (args[10], sr), (args[12], spart)]
        elif name == "ppo_gemm_f32_towers":
            sa, sb, sc, sbias, spre, saux, sbg = args[-7:]
            a_layout, b_layout, A, B, C, pre, aux, bg = args[2], args[3], args[4], args[7], args[9], args[19], \
                args[20], args[22]
            params = [(B, sb)] if b_layout == 1 else []   # input cotangent: dZ W^T
            bufs = ([] if b_layout == 1 else [(B, sb)]) + [(C, sc)] + ([(A, sa)] if sa else [])
            bufs += [(x, s) for x, s in ((pre, spre), (aux, saux), (bg, sbg)) if x]
        else:
            continue
        for ptr, stride in params:
            assert stride == ex.pair and ptr in actor_params and ptr + 4 * stride in critic_params, name
        for ptr, stride in bufs:
            assert inside(ptr, actor_bufs) and inside(ptr + 4 * stride, critic_bufs), name
            checked += 1
    assert checked > 0


class SeqRecurrentExecutor(RecurrentExecutor):
    """The recurrent executor with the one-launch recurrence taken whatever
    the device (its launch sequence only is recorded here)."""

    @staticmethod
    def _seq_fits(Bm, H):
        return True


class SeqRecurrentGemmDwExecutor(SeqRecurrentExecutor):
    """... with the GRU's input projections and weight gradients as GEMMs
    before the forward and after the backward."""
    SEQ_DW = False
    SEQ_XW = False


@pytest.mark.parametrize("fused_dw", [True, False])
def test_recurrent_update_runs_each_direction_of_the_recurrence_in_one_launch(fused_dw):
    r = small(4)
    prog = Program(r.network.plan(r.obs_dim))
    flat = FlatState(prog, torch.device("cpu"))
    cls = SeqRecurrentExecutor if fused_dw else SeqRecurrentGemmDwExecutor
    ex = cls(prog, flat, r.cfg, r.optimizer, r.T, r.N)
    ex.bind(fake_inputs(ex))
    H, I, Bm, T = prog.gru.H, prog.gru.fin, ex.Bm, r.T
    assert ex.seq and ex.seq_dw == ex.seq_xw == (fused_dw and H == 256 and I == 256)
    calls = ex.record()
    names = [n for n, _ in calls]
    steps = r.cfg.update_epochs * r.cfg.num_minibatches
    bwd = "ppo_gru_bwd_seq_dw_f32" if ex.seq_dw else "ppo_gru_bwd_seq_f32"
    fwd = "ppo_gru_fwd_seq_xw_f32" if ex.seq_xw else "ppo_gru_fwd_seq_f32"
    assert names.count(fwd) == steps and names.count(bwd) == steps
    # the input projections' GEMM (into XI) only without the in-launch projections
    xi_gemms = sum(1 for n, a in calls if n == "ppo_gemm_f32" and a[8] == ex.XI.data_ptr())
    assert xi_gemms == (0 if ex.seq_xw else steps)
    assert names.count("ppo_gru_fwd_step_f32") == 2          # the bootstrap's two-step tail
    assert "ppo_gru_bwd_step_f32" not in names
    # every GEMM whose output is a GRU kernel's gradient partial
    dw_out = {ex.WHPART.data_ptr(), ex.WIPART.data_ptr()}
    dw_gemms = sum(1 for n, a in calls if n == "ppo_gemm_f32" and a[8] in dw_out)
    assert dw_gemms == (0 if ex.seq_dw else 2 * steps)
    e_ptr, lde = ex._trunk_out()
    for name, args in calls:
        _, argtypes = _lib.SIGNATURES[name]
        assert len(args) == len(argtypes), name
        if name == "ppo_gru_fwd_seq_f32":
            assert args[3] == Bm * 3 * H and args[10] == Bm and args[-6:-3] == (Bm, H, T)
            assert args[-3] == ex.SEQX.data_ptr() and args[-2] == ex.SEQERR.data_ptr()
        # with both fused launches, one ring per direction: each is zero on entry (no zeroing
        # launch) and its launch zeroes the other direction's ring as it finishes
        pair = ex.SEQX_F is not None
        assert pair == (ex.seq_xw and ex.seq_dw)
        if name == "ppo_gru_fwd_seq_xw_f32":
            assert args[7] == Bm and args[20:23] == (Bm, H, T)
            ring = ex.SEQX_F if pair else ex.SEQX
            assert args[23] == ring.data_ptr() and args[24] == ex.SEQERR.data_ptr()
            assert args[26:30] == (e_ptr, lde, Bm * lde, I)
            assert args[30] == ex.flat.view(prog.gru.wi) and args[31] == 3 * H and args[32] == ex.flat.view(prog.gru.bi)
            assert args[33:] == ((1, ex.SEQX.data_ptr(), 8 * ex.SEQX.numel()) if pair else (0, None, 0))
            if pair:
                assert ex.SEQX_F.numel() == 2 * Bm * H
        if name in ("ppo_gru_bwd_seq_f32", "ppo_gru_bwd_seq_dw_f32"):
            assert args[6] == Bm and args[9] == Bm * H and args[22:25] == (Bm, H, T)
        if name == "ppo_gru_bwd_seq_dw_f32":
            assert args[28:32] == (e_ptr, lde, Bm * lde, I)
            assert args[32:36] == (ex.WHPART.data_ptr(), ex.WHBPART.data_ptr(), ex.WIPART.data_ptr(),
                                   ex.WIBPART.data_ptr())
            assert args[25] == ex.SEQX.data_ptr()
            assert args[36:] == ((1, ex.SEQX_F.data_ptr(), 8 * ex.SEQX_F.numel()) if pair else (0, None, 0))
            assert ex.wh_splits == ex.wi_splits == (Bm + 15) // 16 == ex.WHPART.shape[0] == ex.WIPART.shape[0]
