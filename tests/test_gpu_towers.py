"""Tower-batched launches: the actor and critic towers of an actor-critic
with separate torsos (flax ActorCritic over two Sequential towers, as in
hangar's continuous-control recipes; forward at
boonta/networks/network.py:38-49, backward of jax.value_and_grad at
boonta/algorithms/ppo.py:155-157) run each depth's Dense + LayerNorm
forward, LayerNorm backward, dW and input-cotangent contraction for both
towers in one launch.

Bar: bit-identical to one single-tower launch per tower (each tower's
values come from the same tile code and the same reduction order), and the
whole update with paired towers bit-identical to the update that runs the
towers as separate launches on two streams; the whole update's parity
against the oracle is the Gaussian cases of the learner tests."""
import numpy as np
import pytest
import torch

from boonta_amd import _lib
from boonta_amd.algorithms.ppo import PPO, flat_state_of
from boonta_amd.learner import MLPExecutor
from boonta_amd.random import key as make_key
from ppo_cases import device_transition, make_case

pytestmark = pytest.mark.gpu

A_ROW, A_COL, B_KN, B_NK = 0, 1, 0, 1


def st():
    return torch.cuda.current_stream().cuda_stream


def rnd(g, *shape, scale=1.0):
    return torch.from_numpy((g.standard_normal(shape) * scale).astype(np.float32)).cuda()


def p(t):
    return 0 if t is None else t.data_ptr()


@pytest.mark.parametrize("rows,K,gather,shared", [(2048, 87, True, True), (300, 256, False, False),
                                                  (17, 64, True, False)])
def test_dense_layernorm_forward_towers_equal_single_launches(rows, K, gather, shared):
    g = np.random.default_rng(rows + K)
    F, src = 256, rows + 40
    X = rnd(g, 2, src, K)
    # each tower's parameters in one block (W | bias | gamma | beta), the
    # critic's one block after the actor's: one stride for all of them
    P = rnd(g, 2, K * F + 3 * F, scale=0.1)
    W = P[:, :K * F].view(2, K, F)
    bias, gamma, beta = P[:, K * F:K * F + F], P[:, K * F + F:K * F + 2 * F], P[:, K * F + 2 * F:]
    gamma += 1.0
    I = torch.from_numpy(g.permutation(src)[:rows].astype(np.int32)).cuda() if gather else None
    Z, Y = torch.zeros(2, rows, F, device="cuda"), torch.zeros(2, rows, F, device="cuda")
    mean, rstd = torch.zeros(2, rows, device="cuda"), torch.zeros(2, rows, device="cuda")
    Zs, Ys, ms, rs = (torch.full_like(t, 7.0) for t in (Z, Y, mean, rstd))
    x_stride = 0 if shared else src * K
    for t in range(2):
        xt = X[0] if shared else X[t]
        _lib.call("ppo_gemm_ln_act_fwd_f32", st(), p(xt), K, p(I), p(W[t]), F, p(bias[t]), p(gamma[t]), p(beta[t]),
                  p(Zs[t]), F, p(Ys[t]), F, p(ms[t]), p(rs[t]), rows, K, F, 1e-6, 3)
    _lib.call("ppo_gemm_ln_act_fwd_f32_towers", st(), 2, p(X[0]), K, p(I), p(W[0]), F, p(bias[0]), p(gamma[0]),
              p(beta[0]), p(Z[0]), F, p(Y[0]), F, p(mean[0]), p(rstd[0]), rows, K, F, 1e-6, 3, x_stride,
              P.shape[1], rows * F, rows)
    torch.cuda.synchronize()
    for a, b in ((Z, Zs), (Y, Ys), (mean, ms), (rstd, rs)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("rows,F,act", [(2048, 256, 3), (333, 256, 1), (64, 100, 0)])
def test_layernorm_backward_towers_equal_single_launches(rows, F, act):
    g = np.random.default_rng(rows * 3 + F)
    lib = _lib.load()
    blocks = lib.ppo_layernorm_bwd_blocks(rows)
    dy, z = rnd(g, 2, rows, F), rnd(g, 2, rows, F, scale=2.0)
    zz = z.double()
    mean = zz.mean(-1).float().contiguous()
    rstd = (1.0 / (zz.var(-1, unbiased=False) + 1e-6).sqrt()).float().contiguous()
    gb = rnd(g, 2, 2 * F, scale=0.1)   # each tower's gamma | beta, one stride for both
    gamma, beta = gb[:, :F], gb[:, F:]
    gamma += 1.0
    dz, part = torch.zeros(2, rows, F, device="cuda"), torch.zeros(2, blocks, 2 * F, device="cuda")
    dzs, parts = torch.full_like(dz, 5.0), torch.full_like(part, 5.0)
    for t in range(2):
        _lib.call("ppo_layernorm_act_bwd_f32", st(), p(dy[t]), F, p(z[t]), F, p(mean[t]), p(rstd[t]), p(gamma[t]),
                  p(beta[t]), p(dzs[t]), F, p(parts[t]), rows, F, act)
    _lib.call("ppo_layernorm_act_bwd_f32_towers", st(), 2, p(dy[0]), F, p(z[0]), F, p(mean[0]), p(rstd[0]),
              p(gamma[0]), p(beta[0]), p(dz[0]), F, p(part[0]), rows, F, act, rows * F, rows, 2 * F,
              blocks * 2 * F)
    torch.cuda.synchronize()
    assert torch.equal(dz, dzs) and torch.equal(part, parts)


GEMM_CASES = [
    # (name, a_layout, b_layout, M, N, K, splits, epi, act, gather, shared_a, tile)
    ("forward-silu-pre", A_ROW, B_KN, 2048, 256, 87, 1, 1, 3, True, True, -1),
    ("forward-relu-ragged", A_ROW, B_KN, 301, 130, 77, 1, 1, 1, False, False, 5),
    ("dw-first-layer", A_COL, B_KN, 87, 256, 2048, 16, 0, 0, True, True, -1),
    ("dw-inner", A_COL, B_KN, 256, 256, 2048, 16, 0, 0, False, False, -1),
    ("dw-registers", A_COL, B_KN, 64, 96, 1000, 3, 0, 0, False, False, 7),
    ("dx-dact-silu", A_ROW, B_NK, 2048, 256, 256, 1, 2, 3, False, False, -1),
    ("dx-dact-tanh-128", A_ROW, B_NK, 512, 256, 256, 1, 2, 2, False, False, 0),
    ("dx-store-8wave", A_ROW, B_NK, 1024, 256, 256, 1, 0, 0, False, False, 8),
]


def two(g, shape, fill=None, scale=1.0):
    """Two towers' copies of an operand in one buffer, tower 1 starting at a
    multiple of 4 elements after tower 0: (tower views, element stride)."""
    n = int(np.prod(shape))
    stride = (n + 3) // 4 * 4
    if fill is None:
        flat = torch.from_numpy((g.standard_normal(2 * stride) * scale).astype(np.float32)).cuda()
    else:
        flat = torch.full((2 * stride,), float(fill), device="cuda")
    return [flat[t * stride:t * stride + n].view(*shape) for t in range(2)], stride


@pytest.mark.parametrize("case", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_gemm_towers_equal_single_launches(case):
    _, al, bl, M, N, K, splits, epi, act, gather, shared, tile = case
    g = np.random.default_rng(M * 7 + N * 3 + K)
    # A: [M, K] (layout 0) or [K, M] (layout 1), its gathered axis over `src` rows
    gl = M if al == A_ROW else K
    src = gl + 50 if gather else gl
    a_shape = (src, K) if al == A_ROW else (src, M)
    A, sa = two(g, a_shape)
    if shared:
        A, sa = [A[0], A[0]], 0
    I = torch.from_numpy(g.permutation(src)[:gl].astype(np.int32)).cuda() if gather else None
    b_shape = (K, N) if bl == B_KN else (N, K)
    B, sb = two(g, b_shape, scale=K ** -0.5)
    C, sc = two(g, (splits, M, N), fill=0)
    Cs, _ = two(g, (splits, M, N), fill=3)
    bias, sbias = two(g, (N,), scale=0.1) if epi == 1 else ([None, None], 0)
    pre, spre = two(g, (M, N), fill=0) if epi == 1 and act == 3 else ([None, None], 0)
    pres, _ = two(g, (M, N), fill=3) if pre[0] is not None else ([None, None], 0)
    aux, saux = two(g, (M, N)) if epi == 2 else ([None, None], 0)
    bg, sbg = two(g, (splits, N), fill=0) if al == A_COL else ([None, None], 0)
    bgs, _ = two(g, (splits, N), fill=3) if bg[0] is not None else ([None, None], 0)
    q = lambda t: None if t is None else t.data_ptr()
    for t in range(2):
        _lib.call("ppo_gemm_f32", st(), al, bl, q(A[t]), a_shape[1], q(I), q(B[t]), b_shape[1], q(Cs[t]), N, M, N, K,
                  splits, M * N, epi, q(bias[t]), act, q(pres[t]), q(aux[t]), N, q(bgs[t]), tile)
    _lib.call("ppo_gemm_f32_towers", st(), 2, al, bl, q(A[0]), a_shape[1], q(I), q(B[0]), b_shape[1], q(C[0]), N, M, N,
              K, splits, M * N, epi, q(bias[0]), act, q(pre[0]), q(aux[0]), N, q(bg[0]), tile, sa, sb, sc, sbias,
              spre, saux, sbg)
    torch.cuda.synchronize()
    for t in range(2):
        assert torch.equal(C[t], Cs[t]), t
        if pre[0] is not None:
            assert torch.equal(pre[t], pres[t]), t
        if bg[0] is not None:
            assert torch.equal(bg[t], bgs[t]), t


def test_tower_strides_must_keep_rows_aligned():
    """A stride that is not a multiple of 4 elements is an argument error
    (reported before anything is launched)."""
    X = torch.zeros(2, 64, 64, device="cuda")
    W = torch.zeros(2, 64, 256, device="cuda")
    Z = torch.zeros(2, 64, 256, device="cuda")
    m = torch.zeros(2, 64, device="cuda")
    with pytest.raises(_lib.KernelError, match="bad argument"):
        _lib.call("ppo_gemm_ln_act_fwd_f32_towers", st(), 2, p(X), 64, None, p(W), 256, None, p(W), p(W), p(Z), 256,
                  p(Z), 256, p(m), p(m), 64, 64, 256, 1e-6, 0, 64 * 64, 64 * 256 + 2, 64 * 256, 64)
    with pytest.raises(_lib.KernelError, match="multiples of 4"):
        _lib.call("ppo_gemm_f32_towers", st(), 2, A_ROW, B_KN, p(X), 64, None, p(W), 256, p(Z), 256, 64, 256, 64, 1,
                  0, 0, None, 0, None, None, 0, None, -1, 6, 0, 64 * 256, 0, 0, 0, 0)


class _TwoStreams(MLPExecutor):
    """The executor with tower pairing switched off: each tower's layers run
    as launches of their own, the towers on two streams."""

    def _pair_stride(self, program):
        return 0


class _PerLayer(MLPExecutor):
    """Paired towers issued layer by layer (the whole-chain launches off)."""
    CHAIN = False


class _TwoStreamsPPO(PPO):
    executor_class = _TwoStreams


class _PerLayerPPO(PPO):
    executor_class = _PerLayer


@pytest.mark.parametrize("use_graph", [False, True])
def test_paired_towers_update_equals_two_stream_update(use_graph):
    r, plan, params, tr, roll = make_case(config=3, T=8, N=128, M=4, E=2)
    results = []
    for cls in (_PerLayerPPO, _TwoStreamsPPO):
        alg = cls(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)
        state = alg.init_from_params({"params": params}, r.obs_dim)
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        assert bool(ex.pair) == (cls is _PerLayerPPO) and not ex.chain_ln
        trans = device_transition(tr, roll)
        for k in (1, 2):
            alg.update(state, make_key(k), trans)
        torch.cuda.synchronize()
        results.append((flat_state_of(state).P.cpu().numpy().copy(), ex.LOGS.cpu().numpy().copy()))
    np.testing.assert_array_equal(results[0][0], results[1][0])
    np.testing.assert_array_equal(results[0][1], results[1][1])


class _OneStreamDW(MLPExecutor):
    """The shared trunk's later weight gradients on the main stream."""
    DW_SIDE = False


class _OneStreamDWPPO(PPO):
    executor_class = _OneStreamDW


@pytest.mark.parametrize("use_graph", [False, True])
def test_side_stream_weight_gradients_are_bit_identical(use_graph):
    """The discrete shared-trunk update (two 256-wide layers) with the later
    layer's weight gradient beside its input cotangent on the side stream,
    against the same launches on one stream: parameters and logs bit for bit."""
    r, plan, params, tr, roll = make_case(config=2, T=8, N=512, M=2, E=2)
    results = []
    for cls in (PPO, _OneStreamDWPPO):
        alg = cls(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)
        state = alg.init_from_params({"params": params}, r.obs_dim)
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        assert ex.fused and ex.prog.shared_head and len(ex.trunk) == 2 and ex.DW_SIDE == (cls is PPO)
        trans = device_transition(tr, roll)
        for k in (1, 2):
            alg.update(state, make_key(k), trans)
        torch.cuda.synchronize()
        results.append((flat_state_of(state).P.cpu().numpy().copy(), ex.LOGS.cpu().numpy().copy()))
    np.testing.assert_array_equal(results[0][0], results[1][0])
    np.testing.assert_array_equal(results[0][1], results[1][1])


# ------------------------------------------------------ whole torso chains
def chain_case(g, towers, L, M, K0, gather):
    """Random parameters of `towers` towers of L Dense(256) + LayerNorm layers,
    each tower's parameters in one block (W0 | b0 | gamma0 | beta0 | W1 | ...),
    tower t one block after tower 0."""
    F = 256
    sizes = [(K0 if l == 0 else F) * F + 3 * F for l in range(L)]
    block = sum(sizes)
    P = torch.from_numpy((g.standard_normal((towers, block)) * 0.05).astype(np.float32)).cuda()
    offs, o = [], 0
    for l in range(L):
        K = K0 if l == 0 else F
        offs.append(dict(W=o, b=o + K * F, g=o + K * F + F, be=o + K * F + 2 * F, K=K))
        o += sizes[l]
    for t in range(towers):
        for d in offs:
            P[t, d["g"]:d["g"] + F] += 1.0
    src = M + 30
    X = torch.from_numpy(g.standard_normal((src, K0)).astype(np.float32)).cuda()
    I = torch.from_numpy(g.permutation(src)[:M].astype(np.int32)).cuda() if gather else None
    return P, offs, X, I, block


def ptrs(xs):
    import ctypes
    a = (ctypes.c_void_p * len(xs))(*xs)
    return a, ctypes.cast(a, ctypes.c_void_p).value


@pytest.mark.parametrize("towers,L,M,K0,gather,act", [(2, 4, 2048, 87, True, 3), (1, 4, 4096, 87, False, 3),
                                                      (2, 3, 300, 256, False, 1), (2, 1, 17, 64, True, 2),
                                                      (2, 2, 33, 100, False, 0)])
def test_forward_chain_equals_one_fused_launch_per_layer(towers, L, M, K0, gather, act):
    g = np.random.default_rng(M + 7 * L + K0)
    F = 256
    P, offs, X, I, block = chain_case(g, towers, L, M, K0, gather)
    Z = torch.full((L, towers, M, F), 9.0, device="cuda")
    Y, mean, rstd = torch.full_like(Z, 9.0), torch.full((L, towers, M), 9.0, device="cuda"), \
        torch.full((L, towers, M), 9.0, device="cuda")
    Zs, Ys, ms, rs = (torch.full_like(t, 7.0) for t in (Z, Y, mean, rstd))
    base = P.data_ptr()
    at = lambda key: [base + 4 * d[key] for d in offs]
    keep = [ptrs(at("W")), ptrs(at("b")), ptrs(at("g")), ptrs(at("be")), ptrs([Z[l, 0].data_ptr() for l in range(L)]),
            ptrs([Y[l, 0].data_ptr() for l in range(L)]), ptrs([mean[l, 0].data_ptr() for l in range(L)]),
            ptrs([rstd[l, 0].data_ptr() for l in range(L)])]
    a = [k[1] for k in keep]
    # the transposed kernels of layers 1.. (one pass of the threads covers a
    # workgroup's share at 2048 and 4096 rows; the smaller grids take the loop
    # at the end of the kernel)
    WT = torch.full((max(L - 1, 1), towers, F, F), 3.0, device="cuda")
    kwt = ptrs([0] + [WT[l - 1, 0].data_ptr() for l in range(1, L)])
    _lib.call("ppo_mlp_ln_fwd_f32", st(), towers, L, X.data_ptr(), K0, p(I), M, K0, a[0], F, F, a[1], a[2], a[3],
              a[4], a[5], F, a[6], a[7], 1e-6, act, 0, block, M * F, M, kwt[1], F * F)
    torch.cuda.synchronize()
    for t in range(towers):
        for l in range(1, L):
            o = offs[l]["W"] + t * block
            assert torch.equal(WT[l - 1, t], P.view(-1)[o:o + F * F].view(F, F).t()), (t, l)
    for t in range(towers):
        x, ldx, idx = X.data_ptr(), K0, p(I)
        for l, d in enumerate(offs):
            o = base + 4 * t * block
            _lib.call("ppo_gemm_ln_act_fwd_f32", st(), x, ldx, idx, o + 4 * d["W"], F, o + 4 * d["b"],
                      o + 4 * d["g"], o + 4 * d["be"], Zs[l, t].data_ptr(), F, Ys[l, t].data_ptr(), F,
                      ms[l, t].data_ptr(), rs[l, t].data_ptr(), M, d["K"], F, 1e-6, act)
            x, ldx, idx = Ys[l, t].data_ptr(), F, 0
    torch.cuda.synchronize()
    for a_, b_ in ((Z, Zs), (Y, Ys), (mean, ms), (rstd, rs)):
        assert torch.equal(a_, b_)


def torch_tower(P, offs, X, I, t, block, act, eps=1e-6):
    """float64 torch forward of tower t with every Z kept for its gradient."""
    F = 256
    Pd = P[t].double()
    x = (X[I.long()] if I is not None else X).double()
    acts = {0: lambda u: u, 1: torch.relu, 2: torch.tanh, 3: torch.nn.functional.silu}
    Zs, params = [], []
    for d in offs:
        W = Pd[d["W"]:d["W"] + d["K"] * F].view(d["K"], F).clone().requires_grad_(True)
        b = Pd[d["b"]:d["b"] + F]
        gam = Pd[d["g"]:d["g"] + F].clone().requires_grad_(True)
        bet = Pd[d["be"]:d["be"] + F].clone().requires_grad_(True)
        z = x @ W + b
        z.retain_grad()
        mu = z.mean(-1, keepdim=True)
        var = (z * z).mean(-1, keepdim=True) - mu * mu
        x = acts[act]((z - mu) * torch.rsqrt(var.clamp_min(0) + eps) * gam + bet)
        Zs.append(z)
        params.append((W, gam, bet))
    return x, Zs, params


@pytest.mark.parametrize("towers,L,M,act", [(2, 4, 2048, 3), (2, 3, 300, 1), (1, 2, 50, 2), (2, 1, 16, 0)])
def test_backward_chain_matches_float64_autograd(towers, L, M, act):
    """dZ of every layer and the LayerNorm scale / bias gradients (sum of the
    16-row block partials) against torch float64 autograd through the same
    tower, from the same float32 forward buffers; 1e-5 relative (L2)."""
    g = np.random.default_rng(M * 3 + L)
    F, K0 = 256, 87
    P, offs, X, I, block = chain_case(g, towers, L, M, K0, True)
    lib = _lib.load()
    Z = torch.zeros(L, towers, M, F, device="cuda")
    Y, mean, rstd = torch.zeros_like(Z), torch.zeros(L, towers, M, device="cuda"), \
        torch.zeros(L, towers, M, device="cuda")
    base = P.data_ptr()
    at = lambda key: [base + 4 * d[key] for d in offs]
    lay = lambda T_: [T_[l, 0].data_ptr() for l in range(L)]
    keep = [ptrs(at(k)) for k in ("W", "b", "g", "be")] + [ptrs(lay(T_)) for T_ in (Z, Y, mean, rstd)]
    a = [k[1] for k in keep]
    # the forward also writes the transposed kernels of layers 1..L-1
    WT = torch.zeros(max(L - 1, 1), towers, F, F, device="cuda")
    kwt = ptrs([0] + [WT[l - 1, 0].data_ptr() for l in range(1, L)])
    _lib.call("ppo_mlp_ln_fwd_f32", st(), towers, L, X.data_ptr(), K0, p(I), M, K0, a[0], F, F, a[1], a[2], a[3],
              a[4], a[5], F, a[6], a[7], 1e-6, act, 0, block, M * F, M, kwt[1], F * F)
    dY = torch.from_numpy(g.standard_normal((towers, M, F)).astype(np.float32)).cuda()
    dZ = torch.full((L, towers, M, F), 5.0, device="cuda")
    blocks = lib.ppo_mlp_ln_bwd_blocks(M)
    part = torch.full((L, towers, blocks, 2 * F), 5.0, device="cuda")
    kb = [ptrs(lay(T_)) for T_ in (Z, mean, rstd)] + [ptrs(at("g")), ptrs(at("be")),
                                                      ptrs([0] + [WT[l - 1, 0].data_ptr() for l in range(1, L)]),
                                                      ptrs(lay(dZ)), ptrs(lay(part))]
    b = [k[1] for k in kb]
    _lib.call("ppo_mlp_ln_bwd_f32", st(), towers, L, dY.data_ptr(), F, M, b[0], b[1], b[2], b[3], b[4], b[5], F,
              b[6], F, b[7], act, M * F, M, block, F * F, blocks * 2 * F)
    torch.cuda.synchronize()
    for t in range(towers):
        out, Zs, params = torch_tower(P, offs, X, I, t, block, act)
        # the chain's forward matches the float64 one; the backward starts
        # from the same cotangent
        assert float((Y[L - 1, t].double() - out).norm() / out.norm()) < 1e-5
        out.backward(dY[t].double())
        for l in range(L):
            ref = Zs[l].grad
            got = dZ[l, t].double()
            assert float((got - ref).norm() / ref.norm()) < 1e-5, (t, l)
            _, gam, bet = params[l]
            tot = part[l, t].double().sum(0)
            assert float((tot[:F] - gam.grad).norm() / gam.grad.norm()) < 1e-5, (t, l, "scale")
            assert float((tot[F:] - bet.grad).norm() / bet.grad.norm()) < 1e-5, (t, l, "bias")


@pytest.mark.parametrize("use_graph", [False, True])
def test_chain_update_matches_the_per_layer_update(use_graph):
    """The whole update with the chain launches against the same update issued
    layer by layer (equal but for float32 summation order in the backward):
    parameters after two updates 1e-5 relative (L2), the logged losses 1e-4."""
    r, plan, params, tr, roll = make_case(config=3, T=8, N=128, M=4, E=2)
    results = []
    for cls in (PPO, _PerLayerPPO):
        alg = cls(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)
        state = alg.init_from_params({"params": params}, r.obs_dim)
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        assert ex.chain_ln == (cls is PPO)
        trans = device_transition(tr, roll)
        for k in (1, 2):
            alg.update(state, make_key(k), trans)
        torch.cuda.synchronize()
        results.append((flat_state_of(state).P.cpu().double(), ex.LOGS.cpu().double()))
    (pa, la), (pb, lb) = results
    assert float((pa - pb).norm() / pb.norm()) < 1e-5
    np.testing.assert_allclose(la.numpy(), lb.numpy(), rtol=1e-4, atol=1e-6)


class _SeparateHead(MLPExecutor):
    """The paired chains with the heads + loss as a launch of their own."""
    CHAIN_HEAD = False


class _SeparateHeadPPO(PPO):
    executor_class = _SeparateHead


@pytest.mark.parametrize("use_graph", [False, True])
def test_chain_with_fused_heads_is_bit_identical_to_separate_launches(use_graph):
    """The forward chain that runs both towers' heads + loss on its last
    layer's output (ppo_mlp_ln_fwd_head_loss_f32) against the chain launch
    followed by ppo_head_loss_f32: the same operations on the same values, so
    the parameters and every logged value after two updates are the same
    bits.  Ragged last tile: 500-row minibatches."""
    r, plan, params, tr, roll = make_case(config=3, T=8, N=250, M=4, E=2)
    results = []
    for cls in (PPO, _SeparateHeadPPO):
        alg = cls(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)
        state = alg.init_from_params({"params": params}, r.obs_dim)
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        assert ex.chain_ln and ex._chain_head == (cls is PPO) and ex.mb % 16 != 0
        trans = device_transition(tr, roll)
        for k in (1, 2):
            alg.update(state, make_key(k), trans)
        torch.cuda.synchronize()
        results.append((flat_state_of(state).P.cpu().numpy().copy(), ex.LOGS.cpu().numpy().copy(),
                        ex.STATS.cpu().numpy().copy()))
    for a, b in zip(*results):
        np.testing.assert_array_equal(a, b)


class _UnfusedChains(MLPExecutor):
    """The paired chains' forward (with the heads + loss) and backward as
    separate launches at every step."""
    FWD_BWD_FUSED = False


class _UnfusedChainsPPO(PPO):
    executor_class = _UnfusedChains


@pytest.mark.parametrize("use_graph", [False, True])
def test_fused_forward_backward_chain_is_bit_identical_to_separate_launches(use_graph):
    """From the second optimizer step of an update on, the forward chain with
    the heads + loss and the backward chain run in one launch
    (ppo_mlp_ln_fwd_head_loss_bwd_f32) on the transposed kernels each Adam
    step writes (ppo_adam_clip_wt_f32): the parameters and every logged value
    after two updates are the same bits as with the two launches per step.
    Ragged last tile: 500-row minibatches."""
    r, plan, params, tr, roll = make_case(config=3, T=8, N=250, M=4, E=2)
    results = []
    for cls in (PPO, _UnfusedChainsPPO):
        alg = cls(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)
        state = alg.init_from_params({"params": params}, r.obs_dim)
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        assert ex._fwd_bwd_fused() == (cls is PPO) and ex.mb % 16 != 0
        trans = device_transition(tr, roll)
        for k in (1, 2):
            alg.update(state, make_key(k), trans)
        torch.cuda.synchronize()
        results.append((flat_state_of(state).P.cpu().numpy().copy(), ex.LOGS.cpu().numpy().copy(),
                        ex.STATS.cpu().numpy().copy()))
    for a, b in zip(*results):
        np.testing.assert_array_equal(a, b)
