"""The GRU recurrence of a sequence minibatch in one launch per direction
(ppo_gru_fwd_seq_f32 / _xw_f32, ppo_gru_bwd_seq_f32 / _dw_f32; the loop of
boonta/networks/blocks/rnn.py:34-54 and its backward through time) against
the per-step launches it replaces, whose parity with the oracle is
test_gpu_rnn.py's: bit-identical h, carries, gates, dh and gate cotangents,
gathered initial carries and resets included.  The error path of the
bounded waits is forced from the host (spin limit 0) and must end the launch
with the error word set."""
import numpy as np
import pytest
import torch

from boonta_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
SPIN = 1 << 18


def st():
    return torch.cuda.current_stream().cuda_stream


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def case(B, H, T, seed, reset_p=0.05):
    rng = np.random.default_rng(seed)
    c = dict(B=B, H=H, T=T)
    c["XI"] = dev(rng.standard_normal((T * B, 3 * H)).astype(np.float32))
    c["WH"] = dev((rng.standard_normal((H, 3 * H)) / np.sqrt(H)).astype(np.float32))
    c["BHN"] = dev((0.1 * rng.standard_normal(H)).astype(np.float32))
    c["POOL"] = dev(np.tanh(rng.standard_normal((B + 11, H))).astype(np.float32))
    c["ENVS"] = dev(rng.permutation(B + 11)[:B].astype(np.int32))
    c["TERM"] = dev((rng.random(T * B) < reset_p).astype(np.uint8))
    c["TRUNC"] = dev((rng.random(T * B) < reset_p / 2).astype(np.uint8))
    c["ROWS"] = dev(rng.permutation(T * B).astype(np.int32))   # flags read through the row table
    c["DOUT"] = dev(rng.standard_normal((T * B, H)).astype(np.float32))
    return c


def out_bufs(B, H, T):
    z = lambda *s: torch.full(s, 7.0, device=DEV)
    return dict(HOUT=z(T * B, H), HP=z(T * B, H), GATES=z(T * B, 4 * H), DHS=z(T * B, H), DG=z(T * B, 4 * H))


def run_steps(c, o):
    B, H, T = c["B"], c["H"], c["T"]
    blk, g4 = B * H, 4 * H
    P = lambda k: c[k].data_ptr()
    Q = lambda k: o[k].data_ptr()
    for t in range(T):
        hprev, hrows = (P("POOL"), P("ENVS")) if t == 0 else (Q("HOUT") + 4 * (t - 1) * blk, None)
        _lib.call("ppo_gru_fwd_step_f32", st(), P("XI") + 4 * t * B * 3 * H, 3 * H, hprev, H, hrows, P("TERM"),
                  P("TRUNC"), P("ROWS") + 4 * t * B, P("WH"), 3 * H, P("BHN"), Q("HOUT") + 4 * t * blk, H,
                  Q("HP") + 4 * t * blk, H, Q("GATES") + 4 * t * B * g4, g4, B, H)
    s = T - 1
    _lib.call("ppo_gru_bwd_step_f32", st(), None, 0, None, 0, None, 0, None, 0, None, None, None,
              P("DOUT") + 4 * s * blk, H, Q("GATES") + 4 * s * B * g4, g4, Q("HP") + 4 * s * blk, H,
              Q("DHS") + 4 * s * blk, H, Q("DG") + 4 * s * B * g4, g4, B, H)
    for t in range(T - 1, 0, -1):
        s = t - 1
        _lib.call("ppo_gru_bwd_step_f32", st(), Q("DG") + 4 * (t * B * g4 + H), g4, P("WH"), 3 * H,
                  Q("DHS") + 4 * t * blk, H, Q("GATES") + 4 * (t * B * g4 + 2 * H), g4, P("TERM"), P("TRUNC"),
                  P("ROWS") + 4 * t * B, P("DOUT") + 4 * s * blk, H, Q("GATES") + 4 * s * B * g4, g4,
                  Q("HP") + 4 * s * blk, H, Q("DHS") + 4 * s * blk, H, Q("DG") + 4 * s * B * g4, g4, B, H)


def run_seq(c, o, sync, err, spin=SPIN, backward=True, dw=None):
    """Both sequence launches; dw: the backward with the weight gradients,
    its GRU input rows dw["E"] and partials dw["WHP"], ["WHB"], ["WIP"], ["WIB"]."""
    B, H, T = c["B"], c["H"], c["T"]
    blk, g4 = B * H, 4 * H
    P = lambda k: c[k].data_ptr()
    Q = lambda k: o[k].data_ptr()
    _lib.call("ppo_gru_fwd_seq_f32", st(), P("XI"), 3 * H, B * 3 * H, P("POOL"), H, P("ENVS"), P("TERM"), P("TRUNC"),
              P("ROWS"), B, P("WH"), 3 * H, P("BHN"), Q("HOUT"), H, blk, Q("HP"), H, blk, Q("GATES"), g4, B * g4,
              B, H, T, sync.data_ptr(), err.data_ptr(), spin)
    if backward and dw is None:
        _lib.call("ppo_gru_bwd_seq_f32", st(), P("WH"), 3 * H, P("TERM"), P("TRUNC"), P("ROWS"), B, P("DOUT"), H, blk,
                  Q("GATES"), g4, B * g4, Q("HP"), H, blk, Q("DHS"), H, blk, Q("DG"), g4, B * g4, B, H, T,
                  sync.data_ptr(), err.data_ptr(), spin)
    elif backward:
        I = dw["E"].shape[1]
        _lib.call("ppo_gru_bwd_seq_dw_f32", st(), P("WH"), 3 * H, P("TERM"), P("TRUNC"), P("ROWS"), B, P("DOUT"), H,
                  blk, Q("GATES"), g4, B * g4, Q("HP"), H, blk, Q("DHS"), H, blk, Q("DG"), g4, B * g4, B, H, T,
                  sync.data_ptr(), err.data_ptr(), spin, dw["E"].data_ptr(), I, B * I, I, dw["WHP"].data_ptr(),
                  dw["WHB"].data_ptr(), dw["WIP"].data_ptr(), dw["WIB"].data_ptr(), 0, None, 0)


def sync_bufs(B, H):
    n = _lib.load().ppo_gru_seq_exchange_bytes(B, H) // 8
    # garbage tags: the launch must zero the ring it uses
    return torch.full((n,), 123 << 32, dtype=torch.int64, device=DEV), torch.zeros(1, dtype=torch.int32, device=DEV)


@pytest.mark.parametrize("B,H,T", [(256, 256, 64), (48, 64, 5), (37, 128, 9), (16, 192, 3), (1, 256, 2),
                                   (256, 256, 1)])
def test_sequence_launches_equal_the_step_launches(B, H, T):
    assert (B + 15) // 16 * (H // 16) <= _lib.load().ppo_gru_seq_max_workgroups()
    c = case(B, H, T, seed=B * 31 + H + T)
    ref, got = out_bufs(B, H, T), out_bufs(B, H, T)
    run_steps(c, ref)
    sync, err = sync_bufs(B, H)
    for rep in range(2):   # twice: the second launch finds the first one's tags in the ring
        run_seq(c, got, sync, err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        for k in ("HOUT", "HP", "GATES", "DHS", "DG"):
            assert torch.equal(got[k], ref[k]), (rep, k)


@pytest.mark.parametrize("B,T", [(256, 64), (37, 9), (16, 3), (1, 2), (256, 1)])
def test_backward_with_weight_gradients(B, T):
    """ppo_gru_bwd_seq_dw_f32: dh and the gate cotangents bit-identical to the
    step launches, and its partials summed over the sequence blocks equal to
    the weight and bias gradients of both GRU kernels, dWh = sum_t hp_t^T
    dgate_t[:, H:4H] and dWi = sum_t e_t^T dgate_t[:, 0:3H] (float64 products
    of the same dgate and hp; 16384 rows at the largest case), to rel-L2
    1e-5.  Ragged last block (37 rows), one step, one sequence."""
    H = I = 256
    c = case(B, H, T, seed=B * 7 + T)
    ref, got = out_bufs(B, H, T), out_bufs(B, H, T)
    run_steps(c, ref)
    rng = np.random.default_rng(B + T)
    parts = _lib.load().ppo_gru_seq_dw_parts(B)
    assert parts == (B + 15) // 16
    dw = dict(E=dev(rng.standard_normal((T * B, I)).astype(np.float32)),
              WHP=torch.full((parts, H, 3 * H), 7.0, device=DEV), WHB=torch.full((parts, 3 * H), 7.0, device=DEV),
              WIP=torch.full((parts, I, 3 * H), 7.0, device=DEV), WIB=torch.full((parts, 3 * H), 7.0, device=DEV))
    sync, err = sync_bufs(B, H)
    print(f"bwd seq dw B={B} T={T}", flush=True)
    run_seq(c, got, sync, err, dw=dw)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    for k in ("HOUT", "HP", "GATES", "DHS", "DG"):
        assert torch.equal(got[k], ref[k]), k
    hp = ref["HP"].double().cpu().numpy()
    dg = ref["DG"].double().cpu().numpy()
    e = dw["E"].double().cpu().numpy()
    want = {"WHP": hp.T @ dg[:, H:], "WIP": e.T @ dg[:, :3 * H], "WHB": dg[:, H:].sum(0), "WIB": dg[:, :3 * H].sum(0)}
    for k, w in want.items():
        g = dw[k].double().sum(0).cpu().numpy()
        rel = np.linalg.norm(g - w) / np.linalg.norm(w)
        assert rel < 1e-5, (k, rel)


@pytest.mark.parametrize("B,T", [(256, 64), (37, 9), (16, 3), (1, 2), (256, 1)])
def test_forward_with_input_projections(B, T):
    """ppo_gru_fwd_seq_xw_f32 against ppo_gru_fwd_seq_f32 on the projections
    xi = e Wi + bi made in float64 and rounded once: the launch sums each
    step's products in an order of its own, so h, the carries and the gates
    agree to 2e-5 (absolute; |h| <= 1) rather than bit for bit, through 64
    steps of the recurrence with resets.  Ragged last block, one step, one
    sequence."""
    H = I = 256
    c = case(B, H, T, seed=B * 5 + T)
    rng = np.random.default_rng(B + 3 * T)
    e = rng.standard_normal((T * B, I)).astype(np.float32)
    wi = (rng.standard_normal((I, 3 * H)) / np.sqrt(I)).astype(np.float32)
    bi = (0.1 * rng.standard_normal(3 * H)).astype(np.float32)
    c["XI"] = dev((e.astype(np.float64) @ wi.astype(np.float64) + bi).astype(np.float32))
    E, WI, BI = dev(e), dev(wi), dev(bi)
    ref, got = out_bufs(B, H, T), out_bufs(B, H, T)
    sync, err = sync_bufs(B, H)
    run_seq(c, ref, sync, err, backward=False)
    blk, g4 = B * H, 4 * H
    P = lambda k: c[k].data_ptr()
    Q = lambda k: got[k].data_ptr()
    print(f"fwd seq xw B={B} T={T}", flush=True)
    _lib.call("ppo_gru_fwd_seq_xw_f32", st(), P("POOL"), H, P("ENVS"), P("TERM"), P("TRUNC"), P("ROWS"), B, P("WH"),
              3 * H, P("BHN"), Q("HOUT"), H, blk, Q("HP"), H, blk, Q("GATES"), g4, B * g4, B, H, T, sync.data_ptr(),
              err.data_ptr(), SPIN, E.data_ptr(), I, B * I, I, WI.data_ptr(), 3 * H, BI.data_ptr(), 0, None, 0)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    for k in ("HOUT", "HP", "GATES"):
        diff = float((got[k] - ref[k]).abs().max())
        assert diff < 2e-5, (k, diff)


def test_a_wait_that_gives_up_sets_the_error_word_and_the_launch_ends():
    """Spin limit 0: every wait past the first step gives up at once.  The
    launch completes; the error word is set; step 0 (no wait) is done."""
    B, H, T = 64, 128, 4
    c = case(B, H, T, seed=5)
    ref, got = out_bufs(B, H, T), out_bufs(B, H, T)
    run_steps(c, ref)
    sync, err = sync_bufs(B, H)
    run_seq(c, got, sync, err, spin=0, backward=False)
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    assert torch.equal(got["HOUT"][:B], ref["HOUT"][:B])
    assert torch.equal(got["GATES"][:B], ref["GATES"][:B])
    # later steps were not computed
    assert bool((got["HOUT"][B:] == 7.0).all())


def test_grids_larger_than_the_resident_workgroups_are_rejected():
    lib = _lib.load()
    cus = lib.ppo_gru_seq_max_workgroups()
    B = 16 * (cus // 4 + 1)   # (B / 16) * (64 / 16) workgroups > cus
    sync = torch.zeros(lib.ppo_gru_seq_exchange_bytes(B, 64) // 8, dtype=torch.int64, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    buf = torch.zeros(16, device=DEV)
    with pytest.raises(_lib.KernelError, match="exceed"):
        _lib.call("ppo_gru_fwd_seq_f32", st(), buf.data_ptr(), 192, 0, buf.data_ptr(), 64, None, None, None, None, 0,
                  buf.data_ptr(), 192, buf.data_ptr(), buf.data_ptr(), 64, 0, None, 64, 0, None, 256, 0, B, 64, 2,
                  sync.data_ptr(), err.data_ptr(), SPIN)


@pytest.mark.parametrize("use_graph", [False, True])
def test_recurrent_update_with_sequence_launches_equals_the_step_launches(use_graph):
    """RecurrentPPO.update with each direction of the recurrence in one launch
    (the input projections and weight gradients as GEMMs before and after
    it) against the same update issued step by step: parameters and logs bit
    for bit after two updates, and no wait gave up.  The default update,
    whose forward launch also makes the input projections and whose backward
    launch also multiplies the GRU's weight gradients (summed in other
    orders), against the first:
    the parameter change of the two updates within rel-L2 1e-3 of its norm,
    the logs within 1e-3 (a clip fraction may move by a sample)."""
    from boonta_amd.algorithms.ppo import flat_state_of
    from boonta_amd.algorithms.recurrent_ppo import RecurrentPPO
    from boonta_amd.learner_rnn import RecurrentExecutor
    from boonta_amd.random import key as make_key
    from ppo_cases import device_recurrent_transition, make_recurrent_case

    class StepExecutor(RecurrentExecutor):
        SEQ = False

    class StepPPO(RecurrentPPO):
        executor_class = StepExecutor

    class GemmDwExecutor(RecurrentExecutor):
        SEQ_DW = False
        SEQ_XW = False

    class GemmDwPPO(RecurrentPPO):
        executor_class = GemmDwExecutor

    r, plan, params, tr, roll, extra = make_recurrent_case(4, T=16, N=256, M=4, E=2, seed=3)
    results = {}
    for cls in (GemmDwPPO, StepPPO, RecurrentPPO):
        alg = cls(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)
        state = alg.init_from_params({"params": params}, r.obs_dim)
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        assert ex.seq == (cls is not StepPPO) and ex.seq_dw == ex.seq_xw == (cls is RecurrentPPO)
        p0 = flat_state_of(state).P.cpu().clone()
        trans = device_recurrent_transition(tr, roll, extra)
        for k in (1, 2):
            alg.update(state, make_key(k), trans)
        torch.cuda.synchronize()
        assert not ex.recurrence_error()
        results[cls] = (flat_state_of(state).P.cpu().clone(), ex.LOGS.cpu().clone())
    assert torch.equal(results[GemmDwPPO][0], results[StepPPO][0])
    assert torch.equal(results[GemmDwPPO][1], results[StepPPO][1])
    d_gemm = (results[GemmDwPPO][0] - p0).double()
    d_fused = (results[RecurrentPPO][0] - p0).double()
    rel = float((d_fused - d_gemm).norm() / d_gemm.norm())
    assert rel < 1e-3, rel
    np.testing.assert_allclose(results[RecurrentPPO][1].numpy(), results[GemmDwPPO][1].numpy(), rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("use_graph", [False, True])
def test_an_update_whose_recurrence_gave_up_keeps_its_parameters_and_raises(use_graph):
    """A recurrence forced to give up (spin limit 0, set from the host): the
    update's optimizer steps and count advance write nothing, logs() raises,
    and so does the next update once the error word's copy has landed; the
    update after that runs again."""
    from boonta_amd.algorithms import RecurrenceError
    from boonta_amd.algorithms.ppo import flat_state_of
    from boonta_amd.algorithms.recurrent_ppo import RecurrentPPO
    from boonta_amd.learner_rnn import RecurrentExecutor
    from boonta_amd.random import key as make_key
    from ppo_cases import device_recurrent_transition, make_recurrent_case

    class GivesUp(RecurrentExecutor):
        SEQ_SPIN = 0

    class GivesUpPPO(RecurrentPPO):
        executor_class = GivesUp

    r, plan, params, tr, roll, extra = make_recurrent_case(4, T=16, N=256, M=4, E=2, seed=3)
    alg = GivesUpPPO(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)
    state = alg.init_from_params({"params": params}, r.obs_dim)
    ex = alg.executor(state, r.T, r.N, r.obs_dim)
    assert ex.seq
    flat = flat_state_of(state)
    p0, count0 = flat.P.clone(), int(flat.count.item())
    trans = device_recurrent_transition(tr, roll, extra)
    alg.update(state, make_key(1), trans)
    torch.cuda.synchronize()
    assert ex.recurrence_error()
    assert torch.equal(flat.P, p0)
    assert int(flat.count.item()) == count0
    with pytest.raises(RecurrenceError):
        alg.logs(state, r.T, r.N, r.obs_dim)
    # the next update learns of it from the error word's copy without waiting
    alg.update(state, make_key(2), trans)
    torch.cuda.synchronize()
    with pytest.raises(RecurrenceError):
        alg.update(state, make_key(3), trans)
    # a healthy spin limit: the error word is cleared at the start of the update
    ex.SEQ_SPIN = RecurrentExecutor.SEQ_SPIN
    if use_graph:
        ex.graphs.clear()   # the captured update holds the spin limit it was captured with
    alg.update(state, make_key(4), trans)
    torch.cuda.synchronize()
    assert not ex.recurrence_error()
    assert not torch.equal(flat.P, p0)
    assert int(flat.count.item()) == count0 + r.cfg.update_epochs * r.cfg.num_minibatches
    logs = alg.logs(state, r.T, r.N, r.obs_dim)
    assert all(np.isfinite(v).all() for v in logs.values())


@pytest.mark.parametrize("B,T", [(256, 64), (37, 9)])
def test_ring_per_direction_needs_no_zeroing_launch(B, T):
    """The learner's fused sequence launches with one exchange ring per
    direction (ring_is_zero: no zeroing launch; each launch zeroes the other
    direction's ring as its workgroups finish): the same bits as the launches
    that zero a shared ring first (itself left full of this launch's tags), the
    other ring all zero after each launch, over two forward / backward rounds
    through the same rings."""
    H = I = 256
    c = case(B, H, T, seed=B * 3 + T)
    rng = np.random.default_rng(B + 5 * T)
    E = dev(rng.standard_normal((T * B, I)).astype(np.float32))
    WI = dev((rng.standard_normal((I, 3 * H)) / np.sqrt(I)).astype(np.float32))
    BI = dev((0.1 * rng.standard_normal(3 * H)).astype(np.float32))
    parts = _lib.load().ppo_gru_seq_dw_parts(B)
    blk, g4 = B * H, 4 * H

    def run(o, dw, fwd_ring, bwd_ring, pair, err):
        P = lambda k: c[k].data_ptr()
        Q = lambda k: o[k].data_ptr()
        fclear = (1, bwd_ring.data_ptr(), 8 * bwd_ring.numel()) if pair else (0, None, 0)
        bclear = (1, fwd_ring.data_ptr(), 8 * fwd_ring.numel()) if pair else (0, None, 0)
        _lib.call("ppo_gru_fwd_seq_xw_f32", st(), P("POOL"), H, P("ENVS"), P("TERM"), P("TRUNC"), P("ROWS"), B,
                  P("WH"), 3 * H, P("BHN"), Q("HOUT"), H, blk, Q("HP"), H, blk, Q("GATES"), g4, B * g4, B, H, T,
                  fwd_ring.data_ptr(), err.data_ptr(), SPIN, E.data_ptr(), I, B * I, I, WI.data_ptr(), 3 * H,
                  BI.data_ptr(), *fclear)
        if pair:
            torch.cuda.synchronize()
            assert not bwd_ring.any(), "the forward left the backward's ring unzeroed"
        _lib.call("ppo_gru_bwd_seq_dw_f32", st(), P("WH"), 3 * H, P("TERM"), P("TRUNC"), P("ROWS"), B, P("DOUT"), H,
                  blk, Q("GATES"), g4, B * g4, Q("HP"), H, blk, Q("DHS"), H, blk, Q("DG"), g4, B * g4, B, H, T,
                  bwd_ring.data_ptr(), err.data_ptr(), SPIN, E.data_ptr(), I, B * I, I, dw["WHP"].data_ptr(),
                  dw["WHB"].data_ptr(), dw["WIP"].data_ptr(), dw["WIB"].data_ptr(), *bclear)
        if pair:
            torch.cuda.synchronize()
            assert not fwd_ring.any(), "the backward left the forward's ring unzeroed"

    def bufs():
        return dict(WHP=torch.full((parts, H, 3 * H), 7.0, device=DEV), WHB=torch.full((parts, 3 * H), 7.0, device=DEV),
                    WIP=torch.full((parts, I, 3 * H), 7.0, device=DEV), WIB=torch.full((parts, 3 * H), 7.0, device=DEV))

    ref, dref = out_bufs(B, H, T), bufs()
    sync, err = sync_bufs(B, H)
    run(ref, dref, sync, sync, False, err)
    ring_f = torch.zeros(2 * B * H, dtype=torch.int64, device=DEV)
    ring_b = torch.zeros(_lib.load().ppo_gru_seq_exchange_bytes(B, H) // 8, dtype=torch.int64, device=DEV)
    for rnd in range(2):
        got, dgot = out_bufs(B, H, T), bufs()
        run(got, dgot, ring_f, ring_b, True, err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        for k in ("HOUT", "HP", "GATES", "DHS", "DG"):
            assert torch.equal(got[k], ref[k]), (rnd, k)
        for k in ("WHP", "WHB", "WIP", "WIB"):
            assert torch.equal(dgot[k], dref[k]), (rnd, k)
