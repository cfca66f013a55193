"""Kernel-level parity of the HIP path (through the C ABI) against the oracle
and float64 numpy: GAE, Threefry split and permutations (bit-exact), the
fp32 MFMA GEMM in all layouts with gather / epilogues / split-K, LayerNorm,
the fused loss and clip + Adam."""
import numpy as np
import pytest
import torch

from boonta_amd import _lib
from oracle import gae as ogae
from oracle import nets, ppo, prng

pytestmark = pytest.mark.gpu

DEV = "cuda"


def st():
    return torch.cuda.current_stream().cuda_stream


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


# ------------------------------------------------------------------- GAE
def run_gae(r, te, tr, v, b, gamma, lam, rho=None, c=None, chunks=0):
    T, N = r.shape
    adv = torch.empty(T, N, device=DEV)
    ret = torch.empty(T, N, device=DEV)
    R, V, Bt = dev(r.astype(np.float32)), dev(v.astype(np.float32)), dev(b.astype(np.float32))
    TE, TR = dev(te), dev(tr)
    RHO = dev(rho.astype(np.float32)) if rho is not None else None
    C = dev(c.astype(np.float32)) if c is not None else None
    _lib.call("ppo_gae_f32", st(), R.data_ptr(), TE.data_ptr(), TR.data_ptr(), V.data_ptr(), Bt.data_ptr(),
              None if RHO is None else RHO.data_ptr(), None if C is None else C.data_ptr(), adv.data_ptr(),
              ret.data_ptr(), T, N, gamma, lam, chunks)
    return host(adv), host(ret)


@pytest.mark.parametrize("weighted", [False, True], ids=["gae", "vtrace"])
@pytest.mark.parametrize("chunks", [1, 3])
def test_gae_on_the_reference_known_answer_case(weighted, chunks):
    g = np.random.default_rng(0)
    shape = (6, 3)
    reward, values = g.normal(size=shape), g.normal(size=shape)
    bootstrap = g.normal(size=shape[1:])
    terminated = g.random(shape) < 0.2
    truncated = (g.random(shape) < 0.2) & ~terminated
    rho, c = (g.uniform(0.5, 1.5, shape) if weighted else np.ones(shape) for _ in range(2))
    f = lambda x: x.astype(np.float32).astype(np.float64)
    exp_a, exp_r = ogae.gae(f(reward), terminated, truncated, f(values), f(bootstrap), 0.9, 0.8,
                            rho=f(rho), c=f(c))
    adv, ret = run_gae(reward, terminated, truncated, values, bootstrap, 0.9, 0.8,
                       rho if weighted else None, c if weighted else None, chunks)
    # the reference test's tolerance (tests/test_algorithms.py:193-194)
    np.testing.assert_allclose(adv, exp_a, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ret, exp_r, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("T, N, chunks", [(128, 2048, 0), (128, 2048, 1), (16, 4096, 0), (64, 1024, 0),
                                          (64, 1024, 16), (1, 5, 0), (37, 70, 4)])
def test_gae_at_workload_shapes(T, N, chunks):
    g = np.random.default_rng(T * 1000 + N)
    r = g.normal(size=(T, N)).astype(np.float32)
    v = g.normal(size=(T, N)).astype(np.float32)
    b = g.normal(size=N).astype(np.float32)
    te = g.random((T, N)) < 0.01
    tr = (g.random((T, N)) < 0.005) & ~te
    exp_a, exp_r = ogae.gae(r, te, tr, v, b, 0.99, 0.95)
    adv, ret = run_gae(r, te, tr, v, b, 0.99, 0.95, chunks=chunks)
    np.testing.assert_allclose(adv, exp_a, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(ret, exp_r, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------ permutation
def test_threefry_split_is_bit_exact():
    for seed in (0, 1, 42, 2**31 + 5):
        k = prng.key(seed)
        K = dev(k.view(np.int32))
        out = torch.empty(7, 2, dtype=torch.int32, device=DEV)
        _lib.call("ppo_threefry_split", st(), K.data_ptr(), out.data_ptr(), 7)
        np.testing.assert_array_equal(host(out).view(np.uint32), prng.split(k, 7))


@pytest.mark.parametrize("n", [0, 1, 2, 7, 512, 1024, 1625, 1626, 4095, 4096, 4097, 65536, 262144])
def test_permutation_is_bit_exact(n):
    k = prng.key(1000 + n)
    K = dev(k.view(np.int32))
    out = torch.zeros(max(n, 1), dtype=torch.int32, device=DEV)
    ws = torch.zeros(_lib.load().ppo_permutation_workspace(n), dtype=torch.uint8, device=DEV)
    _lib.call("ppo_permutation", st(), K.data_ptr(), out.data_ptr(), n, ws.data_ptr(), ws.numel())
    got = host(out)[:n]
    np.testing.assert_array_equal(got, prng.permutation(k, n))


@pytest.mark.parametrize("E, n", [(4, 512), (4, 65536), (4, 262144), (4, 1024), (3, 1), (2, 5000), (1, 2000000),
                                  (1, 1 << 23)])
def test_epoch_permutations_are_bit_exact(E, n):
    k = prng.key(7 * n + E)
    K = dev(k.view(np.int32))
    out = torch.zeros(E, n, dtype=torch.int32, device=DEV)
    ws = torch.zeros(_lib.load().ppo_epoch_permutations_workspace(E, n), dtype=torch.uint8, device=DEV)
    _lib.call("ppo_epoch_permutations", st(), K.data_ptr(), E, n, out.data_ptr(), ws.data_ptr(), ws.numel())
    np.testing.assert_array_equal(host(out), prng.epoch_permutations(k, E, n))


# ------------------------------------------------------------------- GEMM
def act_np(name, x):
    return nets.act_fwd(name, x) if name != "none" else x


def gemm_case(a_layout, b_layout, M, N, K, rows_src=None, gather=False, epi=0, act="none", splits=1,
              with_pre=False, bias_grad=False, seed=0, tile=-1):
    g = np.random.default_rng(seed)
    # logical operands A (M x K) and B (K x N), stored per layout
    if a_layout == 0:
        src_rows = rows_src or M
        Astore = g.standard_normal((src_rows, K)).astype(np.float32)
        idx = g.permutation(src_rows)[:M].astype(np.int32) if gather else None
        Alog = Astore[idx] if gather else Astore
    else:
        src_rows = rows_src or K
        Astore = g.standard_normal((src_rows, M)).astype(np.float32)
        idx = g.permutation(src_rows)[:K].astype(np.int32) if gather else None
        Alog = (Astore[idx] if gather else Astore).T
    Blog = g.standard_normal((K, N)).astype(np.float32)
    Bstore = Blog if b_layout == 0 else np.ascontiguousarray(Blog.T)
    bias = g.standard_normal(N).astype(np.float32)
    aux = g.standard_normal((M, N)).astype(np.float32)
    if act in ("relu", "tanh") and epi == 2:
        aux = act_np(act, aux).astype(np.float32)
    A_t, B_t = dev(Astore), dev(Bstore)
    idx_t = dev(idx) if idx is not None else None
    C = torch.zeros(splits, M, N, device=DEV)
    PRE = torch.zeros(M, N, device=DEV) if with_pre else None
    AUX = dev(aux)
    BIAS = dev(bias)
    BG = torch.zeros(splits, N, device=DEV) if bias_grad else None
    lda = Astore.shape[1]
    ldb = Bstore.shape[1]
    _lib.call("ppo_gemm_f32", st(), a_layout, b_layout, A_t.data_ptr(), lda,
              None if idx_t is None else idx_t.data_ptr(), B_t.data_ptr(), ldb, C.data_ptr(), N, M, N, K, splits,
              M * N, epi, BIAS.data_ptr() if epi == 1 else None, _lib.ACT[act],
              None if PRE is None else PRE.data_ptr(), AUX.data_ptr() if epi == 2 else None, N,
              None if BG is None else BG.data_ptr(), tile)
    ref = Alog.astype(np.float64) @ Blog.astype(np.float64)
    got = host(C).sum(0)
    if epi == 1:
        pre = ref + bias
        if with_pre:
            np.testing.assert_allclose(host(PRE), pre, rtol=1e-4, atol=1e-4)
        ref = act_np(act, pre)
        got = host(C)[0]
    elif epi == 2:
        ref = ref * nets.act_bwd(act, aux, aux, np.ones_like(ref)) if act != "none" else ref
        got = host(C)[0]
    scale = np.abs(Alog).astype(np.float64) @ np.abs(Blog).astype(np.float64) + 1.0
    assert np.all(np.abs(got - ref) <= 1e-5 * scale), np.abs(got - ref).max()
    if bias_grad:
        np.testing.assert_allclose(host(BG).sum(0), Blog.astype(np.float64).sum(0), rtol=1e-4, atol=1e-3)
    return C


@pytest.mark.parametrize("a_layout, b_layout", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M, N, K", [(256, 256, 64), (100, 72, 87), (33, 7, 5), (1, 1, 1), (300, 130, 400),
                                     (300, 132, 404), (68, 36, 1000)])
def test_gemm_layouts_match_float64(a_layout, b_layout, M, N, K):
    gemm_case(a_layout, b_layout, M, N, K, seed=M + N + K)


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9])
def test_gemm_every_tile(tile):
    gemm_case(0, 0, 200, 190, 48, tile=tile, seed=tile)
    gemm_case(1, 0, 130, 70, 500, tile=tile, splits=3, bias_grad=True, seed=tile + 10)
    # the input cotangent's layout (B = W^T) with the activation derivative, ragged M and N
    gemm_case(0, 1, 300, 200, 136, epi=2, act="relu", seed=tile + 20, tile=tile)


def test_gemm_forward_gathers_rows():
    gemm_case(0, 0, 512, 256, 400, rows_src=4096, gather=True)
    gemm_case(0, 0, 100, 64, 87, rows_src=1000, gather=True)


@pytest.mark.parametrize("act", ["none", "relu", "tanh", "silu"])
def test_gemm_bias_activation_epilogue(act):
    gemm_case(0, 0, 300, 256, 64, epi=1, act=act, with_pre=True)


@pytest.mark.parametrize("act", ["relu", "tanh", "silu"])
def test_gemm_activation_derivative_epilogue(act):
    gemm_case(0, 1, 300, 256, 136, epi=2, act=act)


@pytest.mark.parametrize("act", ["relu", "silu"])
def test_gemm_activation_derivative_prefetched_aux_is_bit_identical(act):
    """The 64 x 64 tile loads the activation values of its outputs before its
    main loop; ragged M and N (clamped rows and columns) and the same bits as
    the 128 x 128 tile, which reads them in its epilogue."""
    c64 = gemm_case(0, 1, 300, 200, 136, epi=2, act=act, seed=5, tile=3)
    c128 = gemm_case(0, 1, 300, 200, 136, epi=2, act=act, seed=5, tile=0)
    assert torch.equal(c64, c128)


def test_silu_and_its_derivative_on_special_and_extreme_arguments():
    """SiLU x / (1 + exp(-x)) and its derivative s (1 + x (1 - s)) take the
    quotient from the hardware reciprocal with one residual correction: the
    elementwise entry points against float64 over ordinary and extreme
    arguments, and the IEEE results of the division where the exponential
    overflows, the argument is infinite, NaN or a signed zero."""
    rng = np.random.default_rng(11)
    special = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-40, -1e-40, 88.0, -88.0, -103.0, -200.0, 200.0,
                        1.0, -1.0, 1e-20, -1e-20], dtype=np.float32)
    x = np.concatenate([special, (rng.standard_normal(4080) * 6).astype(np.float32),
                        rng.uniform(-90, 90, 4096).astype(np.float32)]).reshape(-1, 64)
    dy = rng.standard_normal(x.shape).astype(np.float32)
    X, DY = dev(x), dev(dy)
    Y, DX = torch.empty_like(X), torch.empty_like(X)
    rows, F = x.shape
    _lib.call("ppo_act_fwd_f32", st(), X.data_ptr(), F, Y.data_ptr(), F, rows, F, _lib.ACT["silu"])
    _lib.call("ppo_act_bwd_f32", st(), DY.data_ptr(), F, X.data_ptr(), F, DX.data_ptr(), F, rows, F, _lib.ACT["silu"])
    y, dx = host(Y).ravel(), host(DX).ravel()
    xs = x.ravel().astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        s = 1.0 / (1.0 + np.exp(-xs))
        y_ref = xs * s
        g_ref = s * (1.0 + xs * (1.0 - s))
    fin = np.isfinite(xs)
    # float32 exp of arguments near 88 carries ~1e-5 relative error from its range reduction, and
    # overflows below -88.7, where SiLU (|y| < 1e-35) comes out as -0
    np.testing.assert_allclose(y[fin], y_ref[fin], rtol=2e-5, atol=1e-35)
    np.testing.assert_allclose(dx[fin], (dy.ravel() * g_ref)[fin], rtol=2e-5, atol=1e-30)
    assert y[0] == np.inf and np.isnan(y[1]) and np.isnan(y[2])
    assert y[3] == 0 and not np.signbit(y[3]) and y[4] == 0 and np.signbit(y[4])
    assert y[10] == 0 and np.signbit(y[10]) and y[11] == 200.0   # exp(200) overflows: -200 / inf = -0
    assert np.isfinite(dx[fin]).all()


@pytest.mark.parametrize("rows, cols, ldx, ldy", [(65536, 87, 87, 88), (5, 3, 7, 8), (1, 4, 4, 12), (300, 1, 1, 4)])
def test_pad_rows_copies_and_zero_fills(rows, cols, ldx, ldy):
    rng = np.random.default_rng(rows + cols)
    X = rng.normal(size=(rows, ldx)).astype(np.float32)
    Y = torch.full((rows, ldy), float("nan"), device=DEV)
    _lib.call("ppo_pad_rows_f32", st(), dev(X).data_ptr(), ldx, Y.data_ptr(), ldy, rows, cols)
    want = np.zeros((rows, ldy), np.float32)
    want[:, :cols] = X[:, :cols]
    assert np.array_equal(host(Y), want)


def test_weight_gradient_over_a_zero_padded_input_matches_the_unpadded_one():
    # the first layer's dW of the paired towers over the padded observation
    # copy (87 -> 88 columns, the copy-fed kernel) against the same contraction
    # on the unpadded rows (the register-staged kernel): the 87 real rows agree
    # to fp32 rounding, the pad row is zero
    rng = np.random.default_rng(7)
    R, F, N, mb, splits = 4096, 87, 256, 2048, 8
    obs = dev(rng.normal(size=(R, F)).astype(np.float32))
    idx = dev(rng.permutation(R)[:mb].astype(np.int32))
    dZ = dev(rng.normal(size=(mb, N)).astype(np.float32))
    pad = torch.zeros(R, 88, device=DEV)
    _lib.call("ppo_pad_rows_f32", st(), obs.data_ptr(), F, pad.data_ptr(), 88, R, F)
    out = {}
    for name, x, ld, M in (("plain", obs, F, F), ("padded", pad, 88, 88)):
        part = torch.zeros(splits, M, N, device=DEV)
        bpart = torch.zeros(splits, N, device=DEV)
        _lib.call("ppo_gemm_f32", st(), 1, 0, x.data_ptr(), ld, idx.data_ptr(), dZ.data_ptr(), N, part.data_ptr(), N,
                  M, N, mb, splits, M * N, 0, None, 0, None, None, 0, bpart.data_ptr(), -1)
        out[name] = host(part).astype(np.float64).sum(0)
    want = host(obs).astype(np.float64)[host(idx)].T @ host(dZ).astype(np.float64)
    np.testing.assert_allclose(out["plain"], want, rtol=2e-5, atol=2e-4)
    np.testing.assert_allclose(out["padded"][:F], want, rtol=2e-5, atol=2e-4)
    assert np.array_equal(out["padded"][F], np.zeros(N))


def test_f32_dw_group_is_bit_identical_to_single_launches():
    import ctypes
    rng = np.random.default_rng(11)
    # (rows of A, M, N, K, splits, gathered): the first layers of the paired
    # towers over the padded observation copy, the later 256-wide layers, and
    # a ragged problem (K not a multiple of the stage depth, M and N not of
    # the tile)
    shapes = [(4096, 88, 256, 2048, 8, True), (4096, 88, 256, 2048, 8, True), (2048, 256, 256, 2048, 4, False),
              (2048, 256, 256, 2048, 4, False), (1000, 68, 132, 1000, 3, False)]
    probs = []
    for R, M, N, K, sp, gathered in shapes:
        A = dev(rng.normal(size=(R, M)).astype(np.float32))
        idx = dev(rng.permutation(R)[:K].astype(np.int32)) if gathered else None
        B = dev(rng.normal(size=(K, N)).astype(np.float32))
        probs.append((A, idx, B, M, N, K, sp))
    single, group = [], []
    for A, idx, B, M, N, K, sp in probs:
        C = torch.full((sp, M, N), float("nan"), device=DEV)
        bg = torch.full((sp, N), float("nan"), device=DEV)
        _lib.call("ppo_gemm_f32", st(), 1, 0, A.data_ptr(), M, None if idx is None else idx.data_ptr(), B.data_ptr(),
                  N, C.data_ptr(), N, M, N, K, sp, M * N, 0, None, 0, None, None, 0, bg.data_ptr(), 3)
        single.append((host(C), host(bg)))
        group.append((torch.full((sp, M, N), float("nan"), device=DEV), torch.full((sp, N), float("nan"), device=DEV)))
    L = len(probs)
    vp = lambda xs: (ctypes.c_void_p * L)(*xs)
    i64 = lambda xs: (ctypes.c_int64 * L)(*xs)
    i32 = lambda xs: (ctypes.c_int * L)(*xs)
    args = [vp([p[0].data_ptr() for p in probs]), i64([p[3] for p in probs]),
            vp([None if p[1] is None else p[1].data_ptr() for p in probs]), vp([p[2].data_ptr() for p in probs]),
            i64([p[4] for p in probs]), vp([c.data_ptr() for c, _ in group]), i64([p[4] for p in probs]),
            i32([p[3] for p in probs]), i32([p[4] for p in probs]), i32([p[5] for p in probs]),
            i32([p[6] for p in probs]), i64([p[3] * p[4] for p in probs]), vp([b.data_ptr() for _, b in group])]
    _lib.call("ppo_gemm_f32_dw_group", st(), L, *[ctypes.addressof(a) for a in args])
    for k, ((c1, b1), (c2, b2)) in enumerate(zip(single, group)):
        assert np.array_equal(c1, host(c2)), f"problem {k}: partials differ"
        assert np.array_equal(b1, host(b2)), f"problem {k}: bias-gradient partials differ"
    # against float64 for the gathered problem
    A, idx, B, M, N, K, sp = probs[0]
    want = host(A).astype(np.float64)[host(idx)].T @ host(B).astype(np.float64)
    np.testing.assert_allclose(single[0][0].astype(np.float64).sum(0), want, rtol=2e-5, atol=2e-4)


@pytest.mark.parametrize("splits", [1, 4, 64])
def test_gemm_split_rows_with_bias_gradient(splits):
    gemm_case(1, 0, 400, 256, 4096, rows_src=8192, gather=True, splits=splits, bias_grad=True)
    gemm_case(1, 0, 256, 8, 2048, splits=splits, bias_grad=True)


# -------------------------------------------------------------- LayerNorm
@pytest.mark.parametrize("F, act", [(256, "silu"), (512, "relu"), (64, "tanh"), (100, "none")])
def test_layernorm_forward_and_backward(F, act):
    g = np.random.default_rng(F)
    rows = 777
    z = g.normal(0.3, 2.0, (rows, F)).astype(np.float32)
    gamma = g.normal(1, 0.2, F).astype(np.float32)
    beta = g.normal(0, 0.2, F).astype(np.float32)
    dy = g.standard_normal((rows, F)).astype(np.float32)
    stages = [{"op": "layernorm", "path": ("ln",), "width": F, "eps": 1e-6}]
    if act != "none":
        stages.append({"op": "act", "fn": act})
    params = {"ln": {"scale": gamma, "bias": beta}}
    y_ref, caches = nets.stages_forward(params, stages, z.astype(np.float64))
    grads = {}
    dz_ref = nets.stages_backward(params, stages, caches, dy.astype(np.float64), grads)
    Z, G, Bt, DY = dev(z), dev(gamma), dev(beta), dev(dy)
    Y = torch.zeros(rows, F, device=DEV)
    mean = torch.zeros(rows, device=DEV)
    rstd = torch.zeros(rows, device=DEV)
    _lib.call("ppo_layernorm_act_fwd_f32", st(), Z.data_ptr(), F, G.data_ptr(), Bt.data_ptr(), Y.data_ptr(), F,
              mean.data_ptr(), rstd.data_ptr(), rows, F, 1e-6, _lib.ACT[act])
    np.testing.assert_allclose(host(Y), y_ref, rtol=1e-4, atol=1e-5)
    blocks = _lib.load().ppo_layernorm_bwd_blocks(rows)
    DZ = torch.zeros(rows, F, device=DEV)
    part = torch.zeros(blocks, 2 * F, device=DEV)
    _lib.call("ppo_layernorm_act_bwd_f32", st(), DY.data_ptr(), F, Z.data_ptr(), F, mean.data_ptr(),
              rstd.data_ptr(), G.data_ptr(), Bt.data_ptr(), DZ.data_ptr(), F, part.data_ptr(), rows, F,
              _lib.ACT[act])
    np.testing.assert_allclose(host(DZ), dz_ref, rtol=1e-4, atol=1e-4)
    p = host(part).sum(0)
    np.testing.assert_allclose(p[:F], grads["ln"]["scale"], rtol=1e-4, atol=1e-3)
    np.testing.assert_allclose(p[F:], grads["ln"]["bias"], rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("rows, K, gather, act", [(2048, 256, False, "silu"), (777, 87, True, "silu"),
                                                   (1, 256, False, "relu"), (33, 64, True, "tanh"),
                                                   (4096, 300, False, "none")])
def test_fused_dense_layernorm_act_forward(rows, K, gather, act):
    """ppo_gemm_ln_act_fwd_f32 against float64 (Dense + LayerNorm + act, the
    oracle's stages) and against the two-launch path it replaces."""
    F = 256
    g = np.random.default_rng(rows + K)
    src_rows = rows + 50 if gather else rows
    x = g.standard_normal((src_rows, K)).astype(np.float32)
    idx = g.permutation(src_rows)[:rows].astype(np.int32) if gather else None
    w = (g.standard_normal((K, F)) / np.sqrt(K)).astype(np.float32)
    b = g.normal(0, 0.1, F).astype(np.float32)
    gamma = g.normal(1, 0.2, F).astype(np.float32)
    beta = g.normal(0, 0.2, F).astype(np.float32)
    stages = [{"op": "dense", "path": ("d",), "in": K, "out": F},
              {"op": "layernorm", "path": ("ln",), "width": F, "eps": 1e-6}]
    if act != "none":
        stages.append({"op": "act", "fn": act})
    params = {"d": {"kernel": w, "bias": b}, "ln": {"scale": gamma, "bias": beta}}
    xs = x[idx] if gather else x
    y_ref, _ = nets.stages_forward(params, stages, xs.astype(np.float64))
    z_ref = xs.astype(np.float64) @ w + b
    X, W, B, G, Bt = dev(x), dev(w), dev(b), dev(gamma), dev(beta)
    I = dev(idx) if gather else None
    Z, Y = torch.zeros(rows, F, device=DEV), torch.zeros(rows, F, device=DEV)
    mean, rstd = torch.zeros(rows, device=DEV), torch.zeros(rows, device=DEV)
    _lib.call("ppo_gemm_ln_act_fwd_f32", st(), X.data_ptr(), K, None if I is None else I.data_ptr(), W.data_ptr(), F,
              B.data_ptr(), G.data_ptr(), Bt.data_ptr(), Z.data_ptr(), F, Y.data_ptr(), F, mean.data_ptr(),
              rstd.data_ptr(), rows, K, F, 1e-6, _lib.ACT[act])
    np.testing.assert_allclose(host(Z), z_ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(host(Y), y_ref, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(host(mean), z_ref.mean(1), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(host(rstd), 1 / np.sqrt(z_ref.var(1) + 1e-6), rtol=1e-4)
    # the two launches it replaces leave the same values
    Z2, Y2 = torch.zeros(rows, F, device=DEV), torch.zeros(rows, F, device=DEV)
    m2, r2 = torch.zeros(rows, device=DEV), torch.zeros(rows, device=DEV)
    _lib.call("ppo_gemm_f32", st(), 0, 0, X.data_ptr(), K, None if I is None else I.data_ptr(), W.data_ptr(), F,
              Z2.data_ptr(), F, rows, F, K, 1, 0, 1, B.data_ptr(), 0, None, None, 0, None, -1)
    _lib.call("ppo_layernorm_act_fwd_f32", st(), Z2.data_ptr(), F, G.data_ptr(), Bt.data_ptr(), Y2.data_ptr(), F,
              m2.data_ptr(), r2.data_ptr(), rows, F, 1e-6, _lib.ACT[act])
    np.testing.assert_allclose(host(Z), host(Z2), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(host(Y), host(Y2), rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------- loss
CFG = {"clip_coefficient": 0.2, "clip_value_loss": True, "entropy_coefficient": 0.01, "value_coefficient": 0.5}


@pytest.mark.parametrize("dist, A, spread", [("categorical", 6, False), ("categorical", 43, False),
                                             ("gaussian", 8, True), ("gaussian", 3, False)])
def test_fused_loss_matches_the_oracle(dist, A, spread):
    g = np.random.default_rng(A)
    rows, B = 3000, 5000
    width = A if (dist == "categorical" or spread) else 2 * A
    ld = width + 2
    head = g.normal(0, 1, (rows, ld)).astype(np.float32)
    value = head[:, width].copy()
    idx = g.permutation(B)[:rows].astype(np.int32)
    if dist == "categorical":
        action = g.integers(0, A, B).astype(np.int32)
    else:
        action = g.standard_normal((B, A)).astype(np.float32)
    scale = g.normal(0, 0.5, A).astype(np.float32) if spread else None
    old_logp = g.normal(-1.5, 0.3, B).astype(np.float32)
    old_value = (g.normal(0, 1, B)).astype(np.float32)
    old_value[idx[:1000]] = value[:1000] + g.normal(0, 0.05, 1000)   # some inside the value clip
    adv = g.normal(0, 1, B).astype(np.float32)
    ret = g.normal(0, 1, B).astype(np.float32)
    # oracle
    h64 = head[:, :width].astype(np.float64)
    if dist == "categorical":
        lp, ent, cache = nets.categorical_stats(h64, action[idx])
    else:
        raw = np.broadcast_to(scale.astype(np.float64), (rows, A)) if spread else h64[:, A:]
        mean = h64[:, :A]
        sig = nets.gaussian_sigma(raw)
        lp, ent = nets.gaussian_stats(mean, sig, action[idx].astype(np.float64))
    old_logp[idx[:500]] = lp[:500].astype(np.float32)   # ratio 1 rows
    loss, logs, (g_lp, g_ent, g_v) = ppo.loss_terms(lp, ent, value.astype(np.float64),
                                                    old_logp[idx].astype(np.float64),
                                                    old_value[idx].astype(np.float64),
                                                    adv[idx].astype(np.float64), ret[idx].astype(np.float64), CFG)
    grads = {}
    if dist == "categorical":
        dhead_ref = nets.categorical_grad(cache, action[idx], g_lp, g_ent)
    else:
        dmean, dsig = nets.gaussian_grad(mean, sig, action[idx].astype(np.float64), g_lp, g_ent)
        draw = dsig / (1 + np.exp(-raw))
        dhead_ref = dmean if spread else np.concatenate([dmean, draw], -1)
        dscale_ref = draw.sum(0)
    # GPU
    H = dev(head)
    DH = torch.zeros(rows, ld, device=DEV)
    blocks = _lib.load().ppo_loss_blocks(rows)
    STATS = torch.zeros(blocks, 11, dtype=torch.float64, device=DEV)
    DS = torch.zeros(blocks, A, device=DEV) if spread else None
    SC = dev(scale) if spread else None
    IDX, ACT = dev(idx), dev(action)
    OLP, OV, ADV, RET = dev(old_logp), dev(old_value), dev(adv), dev(ret)
    _lib.call("ppo_loss_f32", st(), _lib.DIST[dist], rows, IDX.data_ptr(), H.data_ptr(), ld,
              H.data_ptr() + 4 * width, ld, A, None if SC is None else SC.data_ptr(),
              ACT.data_ptr() if dist == "categorical" else None, ACT.data_ptr() if dist == "gaussian" else None,
              OLP.data_ptr(), OV.data_ptr(), ADV.data_ptr(), RET.data_ptr(), DH.data_ptr(),
              DH.data_ptr() + 4 * width, None if DS is None else DS.data_ptr(), STATS.data_ptr(), 0.2, 1, 0.01,
              0.5, 1.0)
    out = torch.zeros(9, device=DEV)
    _lib.call("ppo_loss_finalize", st(), STATS.data_ptr(), blocks, rows, 0.01, 0.5, out.data_ptr())
    dh = host(DH)
    np.testing.assert_allclose(dh[:, :width], dhead_ref, rtol=1e-4, atol=1e-8)
    np.testing.assert_allclose(dh[:, width], g_v, rtol=1e-4, atol=1e-9)
    np.testing.assert_array_equal(dh[:, width + 1:], 0.0)
    o = host(out)
    names = ["actor/loss", "actor/entropy", "actor/approximate_kl", "actor/clip_fraction", "actor/advantage",
             "critic/loss", "critic/explained_variance", "critic/value"]
    for i, n in enumerate(names):
        np.testing.assert_allclose(o[i], logs[n], rtol=1e-5, atol=1e-6, err_msg=n)
    np.testing.assert_allclose(o[8], loss, rtol=1e-5, atol=1e-6)
    if spread:
        np.testing.assert_allclose(host(DS).sum(0), dscale_ref, rtol=1e-4, atol=1e-7)


# ------------------------------------------------------------------- Adam
@pytest.mark.parametrize("nparts", [1, 3, 17, 37, 64, 512])
def test_grad_reduce_partials(nparts):
    """Partial sums of two segments (ragged counts, padded part strides):
    the reduced gradient and its per-chunk squared norms."""
    import struct
    g = np.random.default_rng(nparts)
    chunk = _lib.load().ppo_grad_reduce_chunk_elems()
    specs = [(1000, 1008), (300, 304)]  # (count, part stride)
    segs, chunks, outs, refs, parts32 = b"", b"", [], [], []
    keep = []
    for k, (n, stride) in enumerate(specs):
        parts = (g.standard_normal((nparts, stride)) * 0.1).astype(np.float32)
        P = dev(parts)
        D = torch.full((n,), float("nan"), device=DEV)
        keep += [P, D]
        segs += struct.pack("<QQqqii", D.data_ptr(), P.data_ptr(), n, stride, nparts, 0)
        chunks += b"".join(struct.pack("<iiq", k, len(chunks) // 16 + j, s)
                           for j, s in enumerate(range(0, n, chunk)))
        outs.append(D)
        refs.append(parts[:, :n].astype(np.float64).sum(0))
        parts32.append(np.ascontiguousarray(parts[:, :n]))
    nch = len(chunks) // 16
    SEGS = torch.tensor(list(segs), dtype=torch.uint8, device=DEV)
    CH = torch.tensor(list(chunks), dtype=torch.uint8, device=DEV)
    SQ = torch.zeros(nch, dtype=torch.float64, device=DEV)
    _lib.call("ppo_grad_reduce", st(), SEGS.data_ptr(), CH.data_ptr(), nch, 0, 0, SQ.data_ptr())
    torch.cuda.synchronize()
    tot = 0.0
    for D, ref, p32 in zip(outs, refs, parts32):
        got = host(D).astype(np.float64)
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6 * np.sqrt(nparts))
        # and bit for bit the documented order, in float32: each quarter of the
        # partials in groups of eight added as a fixed tree, quarters in order
        np.testing.assert_array_equal(host(D), reduce_order_f32(p32))
        tot += float((got * got).sum())
    np.testing.assert_allclose(host(SQ).sum(), tot, rtol=1e-12)


def reduce_order_f32(parts):
    """ppo_grad_reduce's sum of partials [nparts, n] in its fixed order, in
    float32 (IEEE round to nearest even, as the kernel's adds)."""
    P, n = parts.shape
    z = np.zeros(n, np.float32)
    t = None
    for w in range(4):
        q0, q1 = P * w // 4, P * (w + 1) // 4
        acc = np.zeros(n, np.float32)
        for q in range(q0, q1, 8):
            v = [parts[q + u] if q + u < q1 else z for u in range(8)]
            acc = acc + (((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7])))
        t = acc if t is None else t + acc
    return t


def test_grad_reduce_few_part_path_is_bit_identical():
    """Chunks of segments with at most ppo_grad_reduce_few_parts() partials,
    put first and counted in nfew, take the wave-per-chunk path: the same
    gradient bits and per-slot squared norms as the block-per-chunk path, for
    1..4 partials, ragged counts, bf16 rounding, signed zeros and a chunk
    count that leaves the last block's waves partly idle."""
    import struct
    lib = _lib.load()
    few_parts = lib.ppo_grad_reduce_few_parts()
    assert few_parts == 4
    g = np.random.default_rng(11)
    chunk = lib.ppo_grad_reduce_chunk_elems()
    specs = [(1, 1000, 1008, 0), (2, 300, 304, 1), (3, 4096 + 256, 4096 + 256, 1), (4, 2060, 2064, 0),
             (3, 36, 40, 0), (7, 520, 520, 0)]  # (nparts, count, part stride, bf16 flag)
    segs, keep, outs, descr = b"", [], [], []
    for k, (npart, n, stride, rb) in enumerate(specs):
        parts = (g.standard_normal((npart, stride)) * 0.1).astype(np.float32)
        parts[:, :8] = 0.0
        parts[0, :4] = -0.0
        P = dev(parts)
        D = torch.full((n,), float("nan"), device=DEV)
        keep += [P]
        outs.append(D)
        segs += struct.pack("<QQqqii", D.data_ptr(), P.data_ptr(), n, stride, npart, rb)
        descr += [(k, s) for s in range(0, n, chunk)]
    slots = {c: i for i, c in enumerate(descr)}
    few = [c for c in descr if specs[c[0]][0] <= few_parts]
    many = [c for c in descr if specs[c[0]][0] > few_parts]
    nch = len(descr)
    SEGS = torch.tensor(list(segs), dtype=torch.uint8, device=DEV)

    def run(order, nfew):
        CH = torch.tensor(list(b"".join(struct.pack("<iiq", k, slots[(k, s)], s) for k, s in order)),
                          dtype=torch.uint8, device=DEV)
        SQ = torch.full((nch,), float("nan"), dtype=torch.float64, device=DEV)
        for D in outs:
            D.fill_(float("nan"))
        _lib.call("ppo_grad_reduce", st(), SEGS.data_ptr(), CH.data_ptr(), nch, nfew, 0, SQ.data_ptr())
        torch.cuda.synchronize()
        return [host(D).view(np.uint32).copy() for D in outs], host(SQ).view(np.uint64).copy()

    ref_g, ref_sq = run(descr, 0)
    got_g, got_sq = run(few + many, len(few))
    assert (len(few) + 3) // 4 * 4 != len(few)  # a partly idle last block
    for k, (a, b) in enumerate(zip(ref_g, got_g)):
        np.testing.assert_array_equal(a, b, err_msg=f"segment {k}")
    np.testing.assert_array_equal(ref_sq, got_sq)
    # an nfew past nchunks is rejected before launch
    with pytest.raises(RuntimeError):
        _lib.call("ppo_grad_reduce", st(), SEGS.data_ptr(), SEGS.data_ptr(), 2, 3, 0, SEGS.data_ptr())
    with pytest.raises(RuntimeError):
        _lib.call("ppo_grad_reduce", st(), SEGS.data_ptr(), SEGS.data_ptr(), 2, 1, 2, SEGS.data_ptr())


def reduce_wide_order_f32(parts):
    """The wide path's order, in float32: sixteen equal partial ranges, each
    in groups of eight added as the fixed tree, the range sums in order."""
    P, n = parts.shape
    z = np.zeros(n, np.float32)
    t = None
    for j in range(16):
        q0, q1 = P * j // 16, P * (j + 1) // 16
        acc = np.zeros(n, np.float32)
        for q in range(q0, q1, 8):
            v = [parts[q + u] if q + u < q1 else z for u in range(8)]
            acc = acc + (((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7])))
        t = acc if t is None else t + acc
    return t


def test_grad_reduce_wide_part_path():
    """Segments with more than ppo_grad_reduce_wide_parts() partials, as the
    last nwide chunks of ppo_grad_reduce_wide_chunk_elems() elements: the
    documented sixteen-range order bit for bit in float32 (ragged counts, a
    bf16-rounded segment), the per-slot squared norms to float64, and a
    middle-path segment and a few-path segment in the same launch unchanged."""
    import struct
    lib = _lib.load()
    wide_parts, wchunk = lib.ppo_grad_reduce_wide_parts(), lib.ppo_grad_reduce_wide_chunk_elems()
    chunk, few_parts = lib.ppo_grad_reduce_chunk_elems(), lib.ppo_grad_reduce_few_parts()
    assert wide_parts == 64 and wchunk == 64
    g = np.random.default_rng(23)
    specs = [(3, 520, 520, 0), (12, 1000, 1008, 0), (64, 1000, 1008, 1), (65, 300, 304, 0), (512, 2304, 2304, 1),
             (130, 36, 40, 0)]
    segs, keep, outs, parts32 = b"", [], [], []
    few, mid, wide = [], [], []
    for k, (npart, n, stride, rb) in enumerate(specs):
        parts = (g.standard_normal((npart, stride)) * 0.05).astype(np.float32)
        P = dev(parts)
        D = torch.full((n,), float("nan"), device=DEV)
        keep.append(P)
        outs.append(D)
        parts32.append(np.ascontiguousarray(parts[:, :n]))
        segs += struct.pack("<QQqqii", D.data_ptr(), P.data_ptr(), n, stride, npart, rb)
        dst = few if npart <= few_parts else wide if npart > wide_parts else mid
        dst += [(k, s) for s in range(0, n, wchunk if dst is wide else chunk)]
    order = few + mid + wide
    nch = len(order)
    SEGS = torch.tensor(list(segs), dtype=torch.uint8, device=DEV)
    CH = torch.tensor(list(b"".join(struct.pack("<iiq", k, i, s) for i, (k, s) in enumerate(order))),
                      dtype=torch.uint8, device=DEV)
    SQ = torch.full((nch,), float("nan"), dtype=torch.float64, device=DEV)
    _lib.call("ppo_grad_reduce", st(), SEGS.data_ptr(), CH.data_ptr(), nch, len(few), len(wide), SQ.data_ptr())
    torch.cuda.synchronize()
    sq = host(SQ)
    for k, ((npart, n, _, rb), D, p32) in enumerate(zip(specs, outs, parts32)):
        got = host(D)
        if npart > wide_parts:
            exp = reduce_wide_order_f32(p32)
        else:
            exp = reduce_order_f32(p32)
        if rb:
            exp = nets.bf16(exp).astype(np.float32)
        np.testing.assert_array_equal(got, exp, err_msg=f"segment {k}")
        for i, (kk, s0) in enumerate(order):
            if kk != k:
                continue
            w = wchunk if npart > wide_parts else chunk
            blk = got[s0:s0 + w].astype(np.float64)
            np.testing.assert_allclose(sq[i], (blk * blk).sum(), rtol=1e-12, err_msg=f"segment {k} chunk {s0}")


@pytest.mark.parametrize("max_norm, scale", [(0.5, 1.0), (0.5, 1e-3), (0.0, 1.0)])
def test_grad_reduce_and_adam_match_optax_restatement(max_norm, scale):
    import struct
    g = np.random.default_rng(int(scale * 1000) + int(max_norm * 10))
    n = 4096 + 64
    nparts = 5
    parts = (g.standard_normal((nparts, n)) * scale * 0.01).astype(np.float32)
    p0 = g.standard_normal(n).astype(np.float32)
    mu0 = (g.standard_normal(n) * 1e-3).astype(np.float32)
    nu0 = (g.random(n) * 1e-5).astype(np.float32)
    P, MU, NU = dev(p0), dev(mu0), dev(nu0)
    Gt = torch.zeros(n, device=DEV)
    PARTS = dev(parts)
    segs = struct.pack("<QQqqii", Gt.data_ptr(), PARTS.data_ptr(), n, n, nparts, 0)
    chunk = _lib.load().ppo_grad_reduce_chunk_elems()
    chunks = b"".join(struct.pack("<iiq", 0, j, s) for j, s in enumerate(range(0, n, chunk)))
    nch = len(range(0, n, chunk))
    SEGS = torch.tensor(list(segs), dtype=torch.uint8, device=DEV)
    CH = torch.tensor(list(chunks), dtype=torch.uint8, device=DEV)
    SQ = torch.zeros(nch, dtype=torch.float64, device=DEV)
    _lib.call("ppo_grad_reduce", st(), SEGS.data_ptr(), CH.data_ptr(), nch, 0, 0, SQ.data_ptr())
    count = torch.tensor([6], dtype=torch.int32, device=DEV)
    _lib.call("ppo_adam_clip_f32", st(), P.data_ptr(), Gt.data_ptr(), MU.data_ptr(), NU.data_ptr(), None, n,
              SQ.data_ptr(), nch, max_norm, 3e-4, 0.9, 0.999, 1e-8, count.data_ptr(), 2, None)
    grad = parts.astype(np.float64).sum(0)
    # absolute floors: fp32 rounding of the operands (|parts| <= ~0.05, |b1 mu| ~ 1e-3,
    # |b2 nu| ~ 1e-5), which exceed the result where terms cancel
    np.testing.assert_allclose(host(Gt), grad, rtol=1e-5, atol=1e-8 * max(scale, 1e-3))
    opt = {"lr": 3e-4, "max_grad_norm": max_norm if max_norm > 0 else None}
    state = {"count": 8, "mu": {"w": mu0.astype(np.float64)}, "nu": {"w": nu0.astype(np.float64)}}
    new, st2, gn = ppo.optimizer_update({"w": grad}, state, {"w": p0.astype(np.float64)}, opt)
    np.testing.assert_allclose(np.sqrt(host(SQ).sum()), gn, rtol=1e-6)
    np.testing.assert_allclose(host(MU), st2["mu"]["w"], rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(host(NU), st2["nu"]["w"], rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(host(P), new["w"], rtol=1e-6, atol=1e-7)
    # the same step from the squared norm folded once (the learner's path)
    SQ1 = torch.zeros(1, dtype=torch.float64, device=DEV)
    _lib.call("ppo_sumsq_total", st(), SQ.data_ptr(), nch, SQ1.data_ptr())
    P2, MU2, NU2 = dev(p0), dev(mu0), dev(nu0)
    _lib.call("ppo_adam_clip_f32", st(), P2.data_ptr(), Gt.data_ptr(), MU2.data_ptr(), NU2.data_ptr(), None, n,
              SQ1.data_ptr(), 1, max_norm, 3e-4, 0.9, 0.999, 1e-8, count.data_ptr(), 2, None)
    np.testing.assert_allclose(host(SQ1)[0], host(SQ).sum(), rtol=1e-14)
    np.testing.assert_allclose(host(P2), new["w"], rtol=1e-6, atol=1e-7)
    # an abort word of zero changes nothing; a nonzero one leaves p, mu, nu (and
    # the bf16 image) as they were, and holds the count
    for word in (0, 3):
        W = torch.tensor([word], dtype=torch.int32, device=DEV)
        P3, MU3, NU3 = dev(p0), dev(mu0), dev(nu0)
        IMG = torch.full((n,), 7, dtype=torch.int16, device=DEV)
        _lib.call("ppo_adam_clip_f32", st(), P3.data_ptr(), Gt.data_ptr(), MU3.data_ptr(), NU3.data_ptr(),
                  IMG.data_ptr(), n, SQ1.data_ptr(), 1, max_norm, 3e-4, 0.9, 0.999, 1e-8, count.data_ptr(), 2,
                  W.data_ptr())
        C = torch.tensor([6], dtype=torch.int32, device=DEV)
        _lib.call("ppo_count_advance", st(), C.data_ptr(), 32, W.data_ptr())
        torch.cuda.synchronize()
        if word == 0:
            assert torch.equal(P3, P2) and int(C.item()) == 38
        else:
            assert np.array_equal(host(P3), p0) and np.array_equal(host(MU3), mu0)
            assert np.array_equal(host(NU3), nu0) and bool((IMG == 7).all()) and int(C.item()) == 6


@pytest.mark.parametrize("n", [0, 1, 1023, 1024, 18700])
def test_sumsq_total_fixed_order(n):
    v = np.random.default_rng(n).random(n)
    V = torch.tensor(v, dtype=torch.float64, device=DEV) if n else torch.zeros(1, dtype=torch.float64, device=DEV)
    T1 = torch.full((1,), 7.0, dtype=torch.float64, device=DEV)
    T2 = torch.full((1,), 7.0, dtype=torch.float64, device=DEV)
    _lib.call("ppo_sumsq_total", st(), V.data_ptr(), n, T1.data_ptr())
    _lib.call("ppo_sumsq_total", st(), V.data_ptr(), n, T2.data_ptr())
    torch.cuda.synchronize()
    np.testing.assert_allclose(host(T1)[0], v.sum(), rtol=1e-13, atol=0)
    assert host(T1)[0] == host(T2)[0]


# ------------------------------------------------------- fused heads + loss
@pytest.mark.parametrize("sep, dist, A, F, rows, act", [
    (False, "categorical", 15, 128, 100, "relu"),     # packed heads, 15 logits + value = 16 outputs
    (True, "gaussian", 4, 64, 197, "tanh"),           # separate towers, state-dependent scale
    (True, "gaussian", 8, 256, 64, "silu"),           # separate towers, state-independent scale
    (True, "categorical", 2, 64, 1, "tanh"),          # a single row
    (False, "categorical", 6, 256, 4099, "none"),     # ragged last tile
    (True, "gaussian", 8, 512, 300, "silu"),          # widest features, 8 blocks per wave
    (False, "categorical", 6, 256, 20000, "relu"),    # above 16384 rows: the 64-row tile kernel
    (False, "categorical", 6, 256, 32768, "tanh"),    # the discrete Anakin minibatch
    (False, "categorical", 15, 256, 16400, "silu"),   # 16 outputs, activation input read separately
    (False, "gaussian", 8, 256, 18000, "relu"),       # shared Gaussian head with a state-independent scale
    (False, "categorical", 6, 128, 16500, "relu"),    # 64-row tiles on 128 features
    (True, "gaussian", 4, 128, 16390, "tanh"),        # ragged 64-row tiles, separate towers
    (True, "gaussian", 8, 256, 17000, "silu"),        # 64-row tiles, activation input read separately
])
def test_fused_heads_loss_and_head_backward(sep, dist, A, F, rows, act):
    g = np.random.default_rng(F + rows + A)
    B = rows + 37
    spread = dist == "gaussian" and F == 256
    width = A if (dist == "categorical" or spread) else 2 * A
    na = width if sep else width + 1
    ldw = (na + 3) // 4 * 4
    z = g.normal(0, 1, (rows, F)).astype(np.float32)          # the torso's last pre-activations
    zc = g.normal(0, 1, (rows, F)).astype(np.float32)
    ha = act_np(act, z).astype(np.float32)
    hc = act_np(act, zc).astype(np.float32) if sep else None
    wa = np.zeros((F, ldw), np.float32)
    wa[:, :na] = g.normal(0, 1 / np.sqrt(F), (F, na))
    ba = np.zeros(ldw, np.float32)
    ba[:na] = g.normal(0, 0.1, na)
    wc = g.normal(0, 1 / np.sqrt(F), (F, 4)).astype(np.float32)
    wc[:, 1:] = 0
    bc = np.array([0.3, 0, 0, 0], np.float32)
    idx = g.permutation(B)[:rows].astype(np.int32)
    action = (g.integers(0, A, B).astype(np.int32) if dist == "categorical"
              else g.standard_normal((B, A)).astype(np.float32))
    scale = g.normal(0, 0.5, A).astype(np.float32) if spread else None
    old_logp = g.normal(-1.5, 0.3, B).astype(np.float32)
    old_value = g.normal(0, 1, B).astype(np.float32)
    adv = g.normal(0, 1, B).astype(np.float32)
    ret = g.normal(0, 1, B).astype(np.float32)
    # oracle: heads in float64, the loss, its cotangents, then the head backward
    ha64, wa64 = ha.astype(np.float64), wa[:, :na].astype(np.float64)
    out = ha64 @ wa64 + ba[:na]
    value = (hc.astype(np.float64) @ wc[:, 0] + bc[0]) if sep else out[:, na - 1]
    if dist == "categorical":
        lp, ent, cache = nets.categorical_stats(out[:, :A], action[idx])
    else:
        raw = np.broadcast_to(scale.astype(np.float64), (rows, A)) if spread else out[:, A:2 * A]
        mean = out[:, :A]
        sig = nets.gaussian_sigma(raw)
        lp, ent = nets.gaussian_stats(mean, sig, action[idx].astype(np.float64))
    loss, logs, (g_lp, g_ent, g_v) = ppo.loss_terms(lp, ent, value, old_logp[idx].astype(np.float64),
                                                    old_value[idx].astype(np.float64),
                                                    adv[idx].astype(np.float64), ret[idx].astype(np.float64), CFG)
    dout = np.zeros((rows, na))
    if dist == "categorical":
        dout[:, :A] = nets.categorical_grad(cache, action[idx], g_lp, g_ent)
    else:
        dmean, dsig = nets.gaussian_grad(mean, sig, action[idx].astype(np.float64), g_lp, g_ent)
        draw = dsig / (1 + np.exp(-raw))
        dout[:, :A] = dmean
        if not spread:
            dout[:, A:2 * A] = draw
    if not sep:
        dout[:, na - 1] = g_v
    def dact(pre, post):
        if act == "none":
            return np.ones_like(pre, np.float64)
        return nets.act_bwd(act, pre.astype(np.float64), post.astype(np.float64), np.ones_like(pre, np.float64))
    # the kernel reads the activation output for relu / tanh and its input for silu
    aux_a, aux_c = (z, zc) if act == "silu" else (ha, hc)
    dha_ref = (dout @ wa64.T) * dact(z, ha)
    dwa_ref = ha64.T @ dout
    # GPU
    HA, WA, BA, WC, BC = dev(ha), dev(wa), dev(ba), dev(wc), dev(bc)
    HC = dev(hc) if sep else None
    XA = dev(aux_a)
    XC = dev(aux_c) if sep else None
    blocks = _lib.load().ppo_head_loss_blocks(rows)
    IDX, ACT = dev(idx), dev(action)
    OLP, OV, ADV, RET = dev(old_logp), dev(old_value), dev(adv), dev(ret)
    SC = dev(scale) if spread else None
    a_code = _lib.ACT[act]
    p = lambda t: None if t is None else t.data_ptr()
    cat = dist == "categorical"

    def launch(records):
        """The kernel's outputs, its per-sample inputs read from separate
        columns or from the 32-byte records of ppo_pack_samples."""
        o = dict(DHA=torch.zeros(rows, F, device=DEV), DHC=torch.zeros(rows, F, device=DEV) if sep else None,
                 WPA=torch.full((blocks, F, ldw), float("nan"), device=DEV),
                 BPA=torch.full((blocks, ldw), float("nan"), device=DEV),
                 WPC=torch.full((blocks, F, 4), float("nan"), device=DEV) if sep else None,
                 BPC=torch.full((blocks, 4), float("nan"), device=DEV) if sep else None,
                 DS=torch.zeros(blocks, A, device=DEV) if spread else None,
                 STATS=torch.zeros(blocks, 11, dtype=torch.float64, device=DEV))
        cols = (OLP.data_ptr(), OV.data_ptr(), ADV.data_ptr(), RET.data_ptr())
        act_i, stride = (ACT.data_ptr() if cat else None), 1
        if records:
            REC = torch.full((B, 8), float("nan"), device=DEV)
            _lib.call("ppo_pack_samples", st(), B, *cols, act_i, REC.data_ptr())
            r = REC.data_ptr()
            cols, act_i, stride = (r, r + 4, r + 8, r + 12), (r + 16 if cat else None), 8
            o["REC"] = REC
        _lib.call("ppo_head_loss_f32", st(), _lib.DIST[dist], rows, IDX.data_ptr(), HA.data_ptr(), F, WA.data_ptr(),
                  ldw, BA.data_ptr(), na, p(HC), F, p(WC) if sep else None, 4, p(BC) if sep else None, F, A, p(SC),
                  act_i, None if cat else ACT.data_ptr(), *cols, a_code, XA.data_ptr(), F,
                  o["DHA"].data_ptr(), F, a_code if sep else 0, p(XC), F, p(o["DHC"]), F, o["WPA"].data_ptr(),
                  o["BPA"].data_ptr(), p(o["WPC"]), p(o["BPC"]), p(o["DS"]), o["STATS"].data_ptr(), 0.2, 1, 0.01, 0.5,
                  1.0, stride)
        return o

    o = launch(False)
    DHA, DHC, WPA, BPA, WPC, BPC, DS, STATS = (o[k] for k in ("DHA", "DHC", "WPA", "BPA", "WPC", "BPC", "DS", "STATS"))
    # the records path: the same values, so the same bits
    r = launch(True)
    torch.cuda.synchronize()
    rec = host(r["REC"])
    np.testing.assert_array_equal(rec[:, :4], np.stack([old_logp, old_value, adv, ret], 1))
    np.testing.assert_array_equal(rec[:, 4].view(np.int32), action if cat else 0)
    np.testing.assert_array_equal(rec[:, 5:], 0.0)
    bits = lambda t: t.view(torch.int64 if t.dtype == torch.float64 else torch.int32)
    for k, t in o.items():
        if t is not None:
            assert torch.equal(bits(t), bits(r[k])), k
    outv = torch.zeros(9, device=DEV)
    _lib.call("ppo_loss_finalize", st(), STATS.data_ptr(), blocks, rows, 0.01, 0.5, outv.data_ptr())
    np.testing.assert_allclose(host(DHA), dha_ref, rtol=1e-4, atol=1e-7)
    wpa = host(WPA).astype(np.float64).sum(0)
    np.testing.assert_allclose(wpa[:, :na], dwa_ref, rtol=1e-4, atol=1e-7)
    np.testing.assert_array_equal(wpa[:, na:], 0.0)
    bpa = host(BPA).astype(np.float64).sum(0)
    np.testing.assert_allclose(bpa[:na], dout.sum(0), rtol=1e-4, atol=1e-7)
    if sep:
        dhc_ref = np.outer(g_v, wc[:, 0]) * dact(zc, hc)
        np.testing.assert_allclose(host(DHC), dhc_ref, rtol=1e-4, atol=1e-8)
        wpc = host(WPC).astype(np.float64).sum(0)
        np.testing.assert_allclose(wpc[:, 0], hc.astype(np.float64).T @ g_v, rtol=1e-4, atol=1e-8)
        np.testing.assert_array_equal(wpc[:, 1:], 0.0)
        np.testing.assert_allclose(host(BPC).astype(np.float64).sum(0)[0], g_v.sum(), rtol=1e-4, atol=1e-8)
    if spread:
        np.testing.assert_allclose(host(DS).astype(np.float64).sum(0), draw.sum(0), rtol=1e-4, atol=1e-7)
    o = host(outv)
    np.testing.assert_allclose(o[8], loss, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(o[1], logs["actor/entropy"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("bf16_image", [False, True])
def test_adam_with_transposed_kernels_is_bit_identical_and_writes_the_transpose(bf16_image):
    """ppo_adam_clip_wt_f32: the same parameters, moments and bf16 image as
    ppo_adam_clip_f32, bit for bit, with each listed 256 x 256 kernel's
    updated values also written transposed (kernels at offsets that are not
    multiples of the block size, with plain elements before, between and after
    them)."""
    import ctypes
    g = np.random.default_rng(21 + bf16_image)
    offs = [260, 260 + 65536 + 1028]
    n = offs[-1] + 65536 + 516
    p0 = g.standard_normal(n).astype(np.float32)
    mu0 = (g.standard_normal(n) * 1e-3).astype(np.float32)
    nu0 = (g.random(n) * 1e-5).astype(np.float32)
    grad = (g.standard_normal(n) * 0.01).astype(np.float32)
    Gt = dev(grad)
    SQ = torch.tensor([float((grad.astype(np.float64) ** 2).sum())], dtype=torch.float64, device=DEV)
    count = torch.tensor([3], dtype=torch.int32, device=DEV)
    outs = []
    for wt in (False, True):
        P, MU, NU = dev(p0), dev(mu0), dev(nu0)
        P16 = torch.zeros(n // 2, dtype=torch.int32, device=DEV) if bf16_image else None
        args = (P.data_ptr(), Gt.data_ptr(), MU.data_ptr(), NU.data_ptr(), P16.data_ptr() if bf16_image else None,
                n, SQ.data_ptr(), 1, 0.5, 3e-4, 0.9, 0.999, 1e-8, count.data_ptr(), 1, None)
        WT = torch.full((len(offs), 256, 256), float("nan"), device=DEV)
        if wt:
            o = (ctypes.c_int64 * 2)(*offs)
            d = (ctypes.c_void_p * 2)(*[WT[r].data_ptr() for r in range(2)])
            _lib.call("ppo_adam_clip_wt_f32", st(), *args, 2, ctypes.addressof(o), ctypes.addressof(d))
        else:
            _lib.call("ppo_adam_clip_f32", st(), *args)
        outs.append((host(P), host(MU), host(NU), host(P16) if bf16_image else None, host(WT)))
    (p1, m1, v1, b1, _), (p2, m2, v2, b2, wt2) = outs
    for a, b in ((p1, p2), (m1, m2), (v1, v2)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    if bf16_image:
        assert np.array_equal(b1, b2)
    assert not np.array_equal(p1, p0)   # the step moved the parameters
    for r, o in enumerate(offs):
        assert np.array_equal(wt2[r].view(np.uint32), p2[o:o + 65536].reshape(256, 256).T.view(np.uint32))
    bad = (ctypes.c_int64 * 2)(offs[0], offs[0] + 256)   # overlapping kernels
    d = (ctypes.c_void_p * 2)(*[WT[r].data_ptr() for r in range(2)])
    P = dev(p0)
    with pytest.raises(_lib.KernelError):
        _lib.call("ppo_adam_clip_wt_f32", st(), P.data_ptr(), Gt.data_ptr(), P.data_ptr(), P.data_ptr(), None, n,
                  SQ.data_ptr(), 1, 0.5, 3e-4, 0.9, 0.999, 1e-8, count.data_ptr(), 1, None, 2,
                  ctypes.addressof(bad), ctypes.addressof(d))
