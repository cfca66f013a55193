"""The bf16 torso chain (ppo_mlp16_ln_fwd) and the packed operand images it
reads (ppo_pack_bf16_operands), on the GPU through the C ABI:

- a packed image holds, chunk by chunk, the MFMA operand layout the header
  states (checked element by element against numpy on the host);
- the chain is bit-identical to the per-layer launches it replaces
  (ppo_splits_bias_act_bf16 + ppo_layernorm_act_fwd_bf16_out16 for the first
  layer; ppo_gemm_bf16s with the rounded bias epilogue +
  ppo_layernorm_act_fwd_bf16_out16 for each later one; ppo_gemm_bf16 for the
  head it can carry): the large-observation trunk (8192 rows, 3 x 512, ReLU,
  two K splits, 44 head outputs), ragged row counts, one split, a single
  layer, heads of 8 to 100 outputs, and the other activations;
- the backward chain (ppo_mlp16_ln_bwd) gives the per-layer launches' dZ16
  bit for bit and their LayerNorm gradient sums to fp32 summation order;
- a whole bf16 PPO.update with the forward chain equals, bit for bit, the same
  update with one launch per layer, and with both chains agrees with it to
  fp32 summation order (the chains' parity with the oracle is that of the
  per-layer path, which test_gpu_bf16 checks; it runs with both chains)."""
import numpy as np
import pytest
import torch

from boonta_amd import _lib
from boonta_amd.algorithms.ppo import flat_state_of
from boonta_amd.learner import ForwardChain
from boonta_amd.random import key as make_key
from ppo_cases import device_transition, gpu_algorithm, make_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
F = 512
EPI_BIAS_ACT = 1


def st():
    return torch.cuda.current_stream().cuda_stream


def bits16(x):
    return x.to(torch.bfloat16).view(torch.int16).contiguous()


def ptrs(ts):
    import ctypes
    arr = (ctypes.c_void_p * len(ts))(*[None if t is None else t.data_ptr() for t in ts])
    return arr, ctypes.cast(arr, ctypes.c_void_p).value


def unpack_reference(W, K, N):
    """The packed layouts restated on the host: fwd chunk kb * (N / 32) + nb
    holds B[16 kb + 8 (l >> 5) + i][32 nb + (l & 31)] at 512 c + 8 l + i for
    B = W; bwd the same for B = W^T."""
    def pack(B):
        KD, ND = B.shape
        out = np.zeros(KD * ND, np.int16)
        l = np.arange(64)
        for kb in range(KD // 16):
            for nb in range(ND // 32):
                c = kb * (ND // 32) + nb
                for i in range(8):
                    out[512 * c + 8 * l + i] = B[16 * kb + 8 * (l >> 5) + i, 32 * nb + (l & 31)]
        return out
    return pack(W), pack(W.T.copy())


@pytest.mark.parametrize("K,N,ldw", [(512, 512, 512), (64, 96, 104)])
def test_pack_bf16_operands_layout(K, N, ldw):
    torch.manual_seed(1)
    Wf = torch.randn(K, ldw, device=DEV)
    W = bits16(Wf)
    fwd = torch.zeros(K * N, dtype=torch.int16, device=DEV)
    bwd = torch.zeros(K * N, dtype=torch.int16, device=DEV)
    wa, wp = ptrs([W])
    fa, fp = ptrs([fwd])
    ba, bp = ptrs([bwd])
    _lib.call("ppo_pack_bf16_operands", st(), 1, wp, ldw, K, N, fp, bp, None, 0, 0, 0, None, None)
    torch.cuda.synchronize()
    ef, eb = unpack_reference(W.cpu().numpy()[:, :N], K, N)
    np.testing.assert_array_equal(fwd.cpu().numpy(), ef)
    np.testing.assert_array_equal(bwd.cpu().numpy(), eb)


def test_pack_head_slot_equals_the_padded_pack():
    """The layers' pack launch with the head in its extra slot gives the
    images ppo_pack_bf16_operand_padded gives."""
    torch.manual_seed(2)
    W = bits16(torch.randn(F, F, device=DEV))
    Wh = bits16(torch.randn(F, 44, device=DEV))
    f1 = torch.zeros(F * F, dtype=torch.int16, device=DEV)
    hf = torch.zeros(F * 64, dtype=torch.int16, device=DEV)
    hb = torch.zeros(F * 64, dtype=torch.int16, device=DEV)
    rf = torch.zeros(F * 64, dtype=torch.int16, device=DEV)
    rb = torch.zeros(F * 64, dtype=torch.int16, device=DEV)
    wa, wp = ptrs([W])
    fa, fp = ptrs([f1])
    _lib.call("ppo_pack_bf16_operands", st(), 1, wp, F, F, F, fp, None, Wh.data_ptr(), 44, 44, 64, hf.data_ptr(),
              hb.data_ptr())
    _lib.call("ppo_pack_bf16_operand_padded", st(), Wh.data_ptr(), 44, F, 44, 64, rf.data_ptr(), rb.data_ptr())
    torch.cuda.synchronize()
    assert torch.equal(hf, rf) and torch.equal(hb, rb)
    ef, eb = unpack_reference(torch.cat([Wh, torch.zeros(F, 20, dtype=torch.int16, device=DEV)], 1).cpu().numpy(),
                              F, 64)
    np.testing.assert_array_equal(hf.cpu().numpy(), ef)
    np.testing.assert_array_equal(hb.cpu().numpy(), eb)


def make_layers(L, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(DEV)
    lay = []
    for l in range(L):
        lay.append(dict(W16=bits16(r(F, F) * 0.05) if l > 0 else None, b=r(F) * 0.1, g=1 + 0.1 * r(F),
                        be=0.1 * r(F)))
    return lay


def per_layer(part, S, M, lay, act, eps=1e-6):
    """The per-layer launches: split sum + bias, then LayerNorm; per later
    layer the bf16 GEMM with the rounded bias epilogue, then LayerNorm."""
    out = []
    for l, p in enumerate(lay):
        Z = torch.zeros(M, F, device=DEV)
        if l == 0:
            _lib.call("ppo_splits_bias_act_bf16", st(), part.data_ptr(), F, M * F, S, p["b"].data_ptr(), 0,
                      Z.data_ptr(), F, M, F)
        else:
            _lib.call("ppo_gemm_bf16s", st(), 0, 0, 1, 1, out[-1]["Y16"].data_ptr(), F, None, p["W16"].data_ptr(),
                      F, Z.data_ptr(), F, M, F, F, 1, 0, EPI_BIAS_ACT, p["b"].data_ptr(), 0, 1, None, 0, None, -1)
        Y = torch.zeros(M, F, device=DEV)
        Y16 = torch.zeros(M, F, dtype=torch.int16, device=DEV)
        mean = torch.zeros(M, device=DEV)
        rstd = torch.zeros(M, device=DEV)
        _lib.call("ppo_layernorm_act_fwd_bf16_out16", st(), Z.data_ptr(), F, p["g"].data_ptr(), p["be"].data_ptr(),
                  Y.data_ptr(), F, Y16.data_ptr(), F, mean.data_ptr(), rstd.data_ptr(), M, F, eps, act)
        out.append(dict(Z=Z, Y=Y, Y16=Y16, mean=mean, rstd=rstd))
    return out


def chain(part, S, M, lay, act, eps=1e-6, y32=None, head=None, z16=False):
    """The chain launch; head = (W16 [512][nh], bias [nh], nh) adds the head
    stage, whose outputs come back as out[-1]["head"]."""
    L = len(lay)
    keep = []
    pk = [None] + [torch.zeros(F * F, dtype=torch.int16, device=DEV) for _ in range(1, L)]
    if L > 1:
        wa, wp = ptrs([p["W16"] for p in lay[1:]])
        fa, fp = ptrs(pk[1:])
        keep += [wa, fa]
        _lib.call("ppo_pack_bf16_operands", st(), L - 1, wp, F, F, F, fp, None, None, 0, 0, 0, None, None)
    out = [dict(Z=(torch.full((M, F), 7, dtype=torch.int16, device=DEV) if z16 else torch.full((M, F), 7.0, device=DEV)),
                Y=torch.full((M, F), 7.0, device=DEV),
                Y16=torch.full((M, F), 7, dtype=torch.int16, device=DEV), mean=torch.full((M,), 7.0, device=DEV),
                rstd=torch.full((M,), 7.0, device=DEV)) for _ in range(L)]
    y32 = [True] * L if y32 is None else y32
    tabs = {}
    for k, src in (("Wp", pk), ("b", [p["b"] for p in lay]), ("g", [p["g"] for p in lay]),
                   ("be", [p["be"] for p in lay]), ("Z", [o["Z"] for o in out]),
                   ("Y", [o["Y"] if y32[l] else None for l, o in enumerate(out)]), ("Y16", [o["Y16"] for o in out]),
                   ("mean", [o["mean"] for o in out]), ("rstd", [o["rstd"] for o in out])):
        a, p = ptrs(src)
        keep.append(a)
        tabs[k] = p
    hargs = (None, None, 0, None, 0)
    if head is not None:
        W16h, bh, nh = head
        npad = (nh + 31) // 32 * 32
        hpk = torch.zeros(F * npad, dtype=torch.int16, device=DEV)
        _lib.call("ppo_pack_bf16_operand_padded", st(), W16h.data_ptr(), nh, F, nh, npad, hpk.data_ptr(), None)
        out[-1]["head"] = torch.full((M, nh), 7.0, device=DEV)
        keep.append(hpk)
        hargs = (hpk.data_ptr(), bh.data_ptr(), nh, out[-1]["head"].data_ptr(), nh)
    _lib.call("ppo_mlp16_ln_fwd", st(), L, part.data_ptr(), F, M * F, S, M, tabs["Wp"], tabs["b"], tabs["g"],
              tabs["be"], tabs["Z"], tabs["Y"], tabs["Y16"], F, tabs["mean"], tabs["rstd"], eps, act, *hargs,
              int(z16))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("M,L,S,act", [(8192, 3, 2, 1), (96, 3, 2, 1), (50, 3, 2, 1), (70, 2, 1, 1), (64, 1, 2, 1),
                                       (64, 2, 2, 3), (64, 2, 2, 2), (33, 2, 3, 0)])
def test_chain_is_bit_identical_to_per_layer_launches(M, L, S, act):
    torch.manual_seed(M + 7 * L + 3 * S + act)
    print(f"chain case M={M} L={L} S={S} act={act}", flush=True)
    part = torch.randn(S, M, F, device=DEV) * 1.5
    lay = make_layers(L, seed=M + L)
    ref = per_layer(part, S, M, lay, act)
    got = chain(part, S, M, lay, act)
    for l in range(L):
        for k in ("Z", "Y", "Y16", "mean", "rstd"):
            assert torch.equal(got[l][k], ref[l][k]), (l, k, (got[l][k] != ref[l][k]).sum().item())


@pytest.mark.parametrize("M,L,nh", [(8192, 3, 44), (50, 2, 44), (64, 1, 8), (96, 3, 64), (33, 2, 100)])
def test_chain_head_is_bit_identical_to_the_head_gemm(M, L, nh):
    """The head stage against ppo_gemm_bf16 on the last layer's fp32 output
    with the bias epilogue, rounded (the per-layer path's head launch)."""
    print(f"chain head case M={M} L={L} nh={nh}", flush=True)
    torch.manual_seed(M + nh)
    part = torch.randn(2, M, F, device=DEV) * 1.5
    lay = make_layers(L, seed=M + 3)
    W16h = bits16(torch.randn(F, nh, device=DEV) * 0.05)
    bh = torch.randn(nh, device=DEV) * 0.1
    got = chain(part, 2, M, lay, 1, head=(W16h, bh, nh))
    ref = per_layer(part, 2, M, lay, 1)
    Wf = W16h.view(torch.bfloat16).float().contiguous()
    H = torch.zeros(M, nh, device=DEV)
    _lib.call("ppo_gemm_bf16", st(), 0, 0, ref[-1]["Y"].data_ptr(), F, None, Wf.data_ptr(), nh, H.data_ptr(), nh, M,
              nh, F, 1, 0, EPI_BIAS_ACT, bh.data_ptr(), 0, 1, None, 0, None, -1)
    torch.cuda.synchronize()
    assert torch.equal(got[-1]["head"], H), (got[-1]["head"] != H).sum().item()
    for k in ("Z", "Y16", "mean", "rstd"):
        assert torch.equal(got[-1][k], ref[-1][k])


@pytest.mark.parametrize("M,L", [(8192, 3), (50, 2)])
def test_chain_bf16_z_is_the_fp32_z_rounded_and_feeds_the_backward_alike(M, L):
    """Z as bf16 (z16): the bit patterns of the fp32 Z (bf16 numbers, so
    exact), every other output unchanged; the backward chain reading it gives
    the same dZ16 and gradient sums as from the fp32 Z."""
    torch.manual_seed(M)
    part = torch.randn(2, M, F, device=DEV) * 1.5
    lay = make_layers(L, seed=M + 9)
    f32 = chain(part, 2, M, lay, 1)
    b16 = chain(part, 2, M, lay, 1, z16=True)
    for l in range(L):
        assert torch.equal(f32[l]["Z"], bits16(f32[l]["Z"]).view(torch.bfloat16).float())
        assert torch.equal(b16[l]["Z"], bits16(f32[l]["Z"]))
        for k in ("Y", "Y16", "mean", "rstd"):
            assert torch.equal(b16[l][k], f32[l][k])
    dY = torch.randn(M, F, device=DEV)
    r32 = bwd_chain(lay, f32, dY, M, 1)
    r16 = bwd_chain(lay, f32, dY, M, 1, z16=True)
    for l in range(L):
        assert torch.equal(r16[l]["dZ16"], r32[l]["dZ16"]) and torch.equal(r16[l]["part"], r32[l]["part"])


def test_chain_without_fp32_outputs_leaves_them_untouched():
    M, L = 64, 3
    part = torch.randn(2, M, F, device=DEV)
    lay = make_layers(L, seed=11)
    ref = per_layer(part, 2, M, lay, 1)
    got = chain(part, 2, M, lay, 1, y32=[False, False, True])
    for l in range(L):
        assert torch.equal(got[l]["Y16"], ref[l]["Y16"]) and torch.equal(got[l]["Z"], ref[l]["Z"])
    assert bool((got[0]["Y"] == 7.0).all()) and bool((got[1]["Y"] == 7.0).all())
    assert torch.equal(got[2]["Y"], ref[2]["Y"])


def test_chain_rejects_bad_arguments():
    part = torch.zeros(2, 32, F, device=DEV)
    a, p = ptrs([None, None])
    # a later layer without its packed operand image
    with pytest.raises(_lib.KernelError, match="ppo_mlp16_ln_fwd"):
        _lib.call("ppo_mlp16_ln_fwd", st(), 2, part.data_ptr(), F, 32 * F, 2, 32, p, p, p, p, p, p, p, F, p, p,
                  1e-6, 1, None, None, 0, None, 0, 0)
    # a head of more outputs than the eight waves' column blocks
    hp = torch.zeros(F * 288, dtype=torch.int16, device=DEV)
    with pytest.raises(_lib.KernelError, match="bad head"):
        _lib.call("ppo_mlp16_ln_fwd", st(), 1, part.data_ptr(), F, 32 * F, 2, 32, p, p, p, p, p, p, p, F, p, p,
                  1e-6, 1, hp.data_ptr(), None, 288, part.data_ptr(), 288, 0)
    # K not a multiple of 32
    with pytest.raises(_lib.KernelError, match="ppo_pack_bf16_operands"):
        _lib.call("ppo_pack_bf16_operands", st(), 1, p, F, 500, F, p, p, None, 0, 0, 0, None, None)


def bwd_inputs(M, L, act, seed):
    """Forward state of an L-layer chain (Z, mean, rstd, Y16 from the forward
    chain on random split partials), kernels and a top cotangent."""
    torch.manual_seed(seed)
    part = torch.randn(2, M, F, device=DEV) * 1.5
    lay = make_layers(L, seed=seed)
    fwd = chain(part, 2, M, lay, act)
    dY = torch.randn(M, F, device=DEV)
    return lay, fwd, dY


def bwd_per_layer(lay, fwd, dY, M, act):
    L = len(lay)
    nb = _lib.load().ppo_layernorm_bwd_blocks(M)
    out = [None] * L
    dy = dY
    for l in range(L - 1, -1, -1):
        dz16 = torch.zeros(M, F, dtype=torch.int16, device=DEV)
        part = torch.zeros(nb, 2 * F, device=DEV)
        _lib.call("ppo_layernorm_act_bwd_bf16_out16", st(), dy.data_ptr(), F, fwd[l]["Z"].data_ptr(), F,
                  fwd[l]["mean"].data_ptr(), fwd[l]["rstd"].data_ptr(), lay[l]["g"].data_ptr(), lay[l]["be"].data_ptr(),
                  dz16.data_ptr(), F, part.data_ptr(), M, F, act)
        out[l] = dict(dZ16=dz16, part=part)
        if l > 0:
            dy = torch.zeros(M, F, device=DEV)
            _lib.call("ppo_gemm_bf16s", st(), 0, 1, 1, 1, dz16.data_ptr(), F, None, lay[l]["W16"].data_ptr(), F,
                      dy.data_ptr(), F, M, F, F, 1, 0, 0, None, 0, 1, None, 0, None, -1)
    torch.cuda.synchronize()
    return out


def bwd_chain(lay, fwd, dY, M, act, head=None, z16=False):
    """The backward chain launch; head = (dhead [M][nh], W16 [512][nh], nh)
    replaces dY by the head's input cotangent."""
    L = len(lay)
    nb = _lib.load().ppo_mlp16_ln_bwd_blocks(M)
    keep = []
    pb = [None] + [torch.zeros(F * F, dtype=torch.int16, device=DEV) for _ in range(1, L)]
    if L > 1:
        wa, wp = ptrs([p["W16"] for p in lay[1:]])
        ba, bp = ptrs(pb[1:])
        keep += [wa, ba]
        _lib.call("ppo_pack_bf16_operands", st(), L - 1, wp, F, F, F, None, bp, None, 0, 0, 0, None, None)
    out = [dict(dZ16=torch.full((M, F), 7, dtype=torch.int16, device=DEV), part=torch.zeros(nb, 2 * F, device=DEV))
           for _ in range(L)]
    tabs = {}
    zs = [bits16(f["Z"]) for f in fwd] if z16 else [f["Z"] for f in fwd]
    keep += zs
    for k, src in (("Wb", pb), ("Z", zs), ("mean", [f["mean"] for f in fwd]),
                   ("rstd", [f["rstd"] for f in fwd]), ("g", [p["g"] for p in lay]), ("be", [p["be"] for p in lay]),
                   ("dZ16", [o["dZ16"] for o in out]), ("part", [o["part"] for o in out])):
        a, p = ptrs(src)
        keep.append(a)
        tabs[k] = p
    hargs = (None, 0, None, 0, 0)
    d16 = (None, 0)
    dy_ptr = dY.data_ptr() if dY is not None else None
    if head is not None:
        dhead, W16h, nh = head
        npad = (nh + 31) // 32 * 32
        hpk = torch.zeros(2, F * npad, dtype=torch.int16, device=DEV)
        _lib.call("ppo_pack_bf16_operand_padded", st(), W16h.data_ptr(), nh, F, nh, npad, hpk[0].data_ptr(),
                  hpk[1].data_ptr())
        keep.append(hpk)
        hargs = (dhead.data_ptr(), nh, hpk[1].data_ptr(), nh, npad)
        dy_ptr = None
        ld16 = (nh + 7) // 8 * 8
        out[0]["dhead16"] = torch.full((M, ld16), 7, dtype=torch.int16, device=DEV)
        d16 = (out[0]["dhead16"].data_ptr(), ld16)
    _lib.call("ppo_mlp16_ln_bwd", st(), L, dy_ptr, F, M, tabs["Wb"], tabs["Z"], tabs["mean"], tabs["rstd"],
              tabs["g"], tabs["be"], tabs["dZ16"], F, tabs["part"], act, *hargs, int(z16), *d16)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("M,L,act", [(8192, 3, 1), (96, 3, 1), (50, 3, 1), (64, 1, 1), (64, 2, 3), (64, 2, 2),
                                     (33, 2, 0)])
def test_backward_chain_matches_per_layer_launches(M, L, act):
    """dZ16 bit for bit (the input cotangents between layers are the bf16
    GEMM's, bit for bit, or dZ16 below the top would differ); the LayerNorm
    gradient sums over all rows to fp32 summation order (the chain sums its
    own 32-row blocks)."""
    print(f"backward chain case M={M} L={L} act={act}", flush=True)
    lay, fwd, dY = bwd_inputs(M, L, act, seed=M + L + act)
    ref = bwd_per_layer(lay, fwd, dY, M, act)
    got = bwd_chain(lay, fwd, dY, M, act)
    for l in range(L):
        assert torch.equal(got[l]["dZ16"], ref[l]["dZ16"]), (l, (got[l]["dZ16"] != ref[l]["dZ16"]).sum().item())
        g = got[l]["part"].double().sum(0).cpu().numpy()
        r = ref[l]["part"].double().sum(0).cpu().numpy()
        scale = ref[l]["part"].double().abs().sum(0).cpu().numpy() + 1e-30
        assert np.all(np.abs(g - r) <= 1e-5 * scale), (l, np.max(np.abs(g - r) / scale))


@pytest.mark.parametrize("M,L,nh", [(8192, 3, 44), (50, 2, 44), (64, 1, 8), (96, 3, 64)])
def test_backward_chain_head_cotangent_matches_the_head_gemm(M, L, nh):
    """The top cotangent from the head (the bf16 head GEMM's dhead W^T,
    rounded) then the chain: dZ16 of every layer bit for bit against the head
    GEMM followed by the per-layer launches."""
    print(f"backward chain head case M={M} L={L} nh={nh}", flush=True)
    lay, fwd, _ = bwd_inputs(M, L, 1, seed=M + nh)
    torch.manual_seed(nh)
    dhead = torch.randn(M, nh, device=DEV) * 0.01
    W16h = bits16(torch.randn(F, nh, device=DEV) * 0.05)
    Wf = W16h.view(torch.bfloat16).float().contiguous()
    dY = torch.zeros(M, F, device=DEV)
    _lib.call("ppo_gemm_bf16", st(), 0, 1, dhead.data_ptr(), nh, None, Wf.data_ptr(), nh, dY.data_ptr(), F, M, F, nh,
              1, 0, 0, None, 0, 1, None, 0, None, -1)
    ref = bwd_per_layer(lay, fwd, dY, M, 1)
    got = bwd_chain(lay, fwd, None, M, 1, head=(dhead, W16h, nh))
    for l in range(L):
        assert torch.equal(got[l]["dZ16"], ref[l]["dZ16"]), (l, (got[l]["dZ16"] != ref[l]["dZ16"]).sum().item())
    # the bf16 copy of the head cotangents: dhead rounded to nearest even, zero past nh
    d16 = got[0]["dhead16"]
    exp = torch.zeros_like(d16)
    exp[:, :nh] = bits16(dhead[:, :nh])
    assert torch.equal(d16, exp)


def run_update(monkeypatch, chain16, bwd=True):
    monkeypatch.setattr(ForwardChain, "CHAIN16", chain16)
    monkeypatch.setattr(ForwardChain, "CHAIN16_BWD", bwd)
    r, plan, params, tr, roll = make_case(config=5, T=8, N=64, M=2, E=2)
    alg = gpu_algorithm(r, use_graph=False)
    state = alg.init_from_params({"params": params}, r.obs_dim)
    trans = device_transition(tr, roll)
    alg.update(state, make_key(3), trans)
    torch.cuda.synchronize()
    ex = alg.executor(state, r.T, r.N, r.obs_dim)
    assert (ex.trunk[0].chain16 is not None) == chain16
    flat = flat_state_of(state)
    logs = alg.logs(state, r.T, r.N, r.obs_dim)
    return flat.P.clone(), flat.MU.clone(), flat.NU.clone(), logs


def test_update_with_forward_chain_equals_per_layer_update(monkeypatch):
    P1, MU1, NU1, logs1 = run_update(monkeypatch, True, bwd=False)
    P0, MU0, NU0, logs0 = run_update(monkeypatch, False)
    assert torch.equal(P1, P0) and torch.equal(MU1, MU0) and torch.equal(NU1, NU0)
    for k in logs0:
        np.testing.assert_array_equal(logs1[k], logs0[k], err_msg=k)


def first_step_gradient(monkeypatch, chain16, bwd):
    monkeypatch.setattr(ForwardChain, "CHAIN16", chain16)
    monkeypatch.setattr(ForwardChain, "CHAIN16_BWD", bwd)
    r, plan, params, tr, roll = make_case(config=5, T=8, N=64, M=2, E=2)
    alg = gpu_algorithm(r, use_graph=False)
    state = alg.init_from_params({"params": params}, r.obs_dim)
    trans = device_transition(tr, roll)
    ex = alg.executor(state, r.T, r.N, r.obs_dim)
    ex.KEY.copy_(torch.from_numpy(make_key(3).view(np.int32).copy()))
    ex.bind(alg._inputs(trans, r.obs_dim)[0])
    ex.issue(torch.cuda.current_stream().cuda_stream, max_steps=1)
    torch.cuda.synchronize()
    return flat_state_of(state).G.clone(), ex


def test_gradient_with_both_chains_matches_per_layer_launches(monkeypatch):
    """The first step's gradient: every Dense gradient bit for bit (their
    operands dZ16 and Y16 are), the LayerNorm scale and bias gradients to
    fp32 summation order (the backward chain sums 32-row blocks)."""
    G1, ex = first_step_gradient(monkeypatch, True, True)
    G0, _ = first_step_gradient(monkeypatch, False, False)
    ln = torch.zeros_like(G0, dtype=torch.bool)
    for lb in ex.trunk:
        for k in ("scale", "bias"):
            reg = lb.spec.ln[k]
            ln[reg.offset:reg.offset + lb.spec.fout] = True
    assert torch.equal(G1[~ln], G0[~ln])
    a, b = G1[ln].double(), G0[ln].double()
    assert ((a - b).abs() <= 1e-5 * b.abs().max() + 1e-5 * b.abs()).all(), (a - b).abs().max().item()
