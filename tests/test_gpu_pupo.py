"""Parity of RecurrentPuPO.update (boonta/algorithms/recurrent_pupo.py:100-308)
on the HIP learner against the oracle's restatement (oracle/ppo.py
recurrent_pupo_update) on the same seeded recurrent rollout.

Each step's env draw is jax.random.choice on probabilities formed from that
step's V-trace advantages; the GPU's float32 advantages and the oracle's
float64 ones agree to about 1e-6, so a draw that lands within that of a
cumulative boundary may pick the neighbouring env.  The oracle therefore
follows the GPU's draws (teacher-forced indices) and the test checks the
oracle's own draw equals the GPU's wherever it lies more than 1e-5 of the
total from a boundary (at least 99 % of draws).

Tolerances (written here): bootstrap 1e-5 relative; importance weights 1e-4
relative; parameters after the update and the first step's gradient 1e-4
relative (L2 per leaf); the carried ratio after the update 1e-4 relative
(L2); logged scalars of every step 1e-5 relative (atol 1e-6; the mean
importance weight 1e-5); graph replay bit-identical to the eager update.
"""
import numpy as np
import pytest
import torch

from boonta_amd.algorithms import RecurrentPuPO, RecurrentPuPOConfig
from boonta_amd.algorithms.ppo import flat_state_of
from boonta_amd.flat import tree_from_flat, tree_to_numpy
from boonta_amd.optim import constant_schedule
from boonta_amd.random import key as make_key
from oracle import ppo
from ppo_cases import device_recurrent_transition, make_recurrent_case, oracle_cfg, oracle_opt, rel_l2, to64

pytestmark = pytest.mark.gpu

CASES = {
    "reduced": dict(T=8, N=64, M=4, E=2),
    "reduced-clipped": dict(T=12, N=48, M=3, E=2),
}
PUPO = {"reduced": dict(), "reduced-clipped": dict(advantage_clip=0.9, trace_clip=0.8, normalize_advantage=False)}


def pupo_cfg(r, **kw) -> RecurrentPuPOConfig:
    c = r.cfg
    return RecurrentPuPOConfig(num_minibatches=c.num_minibatches, update_epochs=c.update_epochs,
                               clip_coefficient=c.clip_coefficient, clip_value_loss=c.clip_value_loss,
                               entropy_coefficient=c.entropy_coefficient, value_coefficient=c.value_coefficient,
                               gamma=c.gamma, gae_lambda=c.gae_lambda, **kw)


def oracle_pupo_cfg(cfg: RecurrentPuPOConfig) -> dict:
    d = oracle_cfg(cfg)
    d.update(advantage_clip=cfg.advantage_clip, trace_clip=cfg.trace_clip,
             priority_exponent=cfg.priority_exponent, normalize_advantage=cfg.normalize_advantage)
    return d


def leaves(tree):
    return dict(ppo.tree_leaves(tree))


def run_gpu(r, cfg, params, trans, key, beta, use_graph=False, max_steps=None, updates=1):
    alg = RecurrentPuPO(cfg=cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph,
                        importance_exponent=constant_schedule(beta))
    state = alg.init_from_params({"params": params}, r.obs_dim)
    if max_steps is None:
        for u in range(updates):
            alg.update(state, key if u == 0 else make_key(1000 + u), trans)
    else:
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        ex.beta = beta
        ex.KEY.copy_(torch.from_numpy(key.view(np.int32).copy()))
        ex.bind(alg._inputs(trans, r.obs_dim)[0])
        ex.issue(torch.cuda.current_stream().cuda_stream, max_steps=max_steps)
    torch.cuda.synchronize()
    return alg, state


@pytest.mark.parametrize("name", list(CASES))
def test_pupo_update_matches_the_oracle(name):
    r, plan, params, tr, roll, extra = make_recurrent_case(4, **CASES[name])
    cfg = pupo_cfg(r, **PUPO[name])
    beta, key = 0.4, make_key(21)
    print(f"\npupo update {name}: T={r.T} N={r.N} M={cfg.num_minibatches} E={cfg.update_epochs}", flush=True)
    alg, state = run_gpu(r, cfg, params, device_recurrent_transition(tr, roll, extra), key, beta)
    ex = alg.executor(state, r.T, r.N, r.obs_dim)
    idx = ex.IDX.cpu().numpy()
    w = ex.WEIGHTS.cpu().numpy()
    p_or, _, info = ppo.recurrent_pupo_update(to64(params), ppo.optimizer_init(to64(params)), plan,
                                              oracle_pupo_cfg(cfg), oracle_opt(r.optimizer), tr, key, beta,
                                              indices=list(idx))
    np.testing.assert_allclose(ex.BOOT.cpu().numpy(), info["bootstrap"], rtol=1e-5, atol=1e-6)
    own, margin = np.stack(info["own_indices"]), np.stack(info["margins"])
    far = margin > 1e-5
    assert far.mean() >= 0.99
    np.testing.assert_array_equal(idx[far], own[far])
    assert idx.min() >= 0 and idx.max() < r.N
    np.testing.assert_allclose(w, np.stack(info["weights"]), rtol=1e-4)
    p_gpu = leaves(tree_to_numpy(state.params["params"]))
    worst = 0.0
    for path, p in leaves(p_or).items():
        err = rel_l2(p_gpu[path], p)
        worst = max(worst, err)
        assert err <= 1e-4, (path, err)
    assert rel_l2(ex.RATIO.cpu().numpy(), info["ratio"]) <= 1e-4
    logs = alg.logs(state, r.T, r.N, r.obs_dim)
    for i, lg in enumerate(info["logs"]):
        for k, v in lg.items():
            if k == "grad_norm":
                continue
            np.testing.assert_allclose(logs[k][i], v, rtol=1e-5, atol=1e-6, err_msg=f"step {i} {k}")
    assert int(flat_state_of(state).count.item()) == cfg.update_epochs * cfg.num_minibatches
    print(f"pupo {name}: worst parameter rel-L2 {worst:.2e}, {int((~far).sum())} draws near a boundary",
          flush=True)


def test_pupo_first_step_at_the_recurrent_workload_size():
    """64 steps x 1024 envs drawing 4 minibatches of 256 envs: the first
    step's env draw, weights, gradient and scattered ratio."""
    r, plan, params, tr, roll, extra = make_recurrent_case(4)
    cfg = pupo_cfg(r)
    beta, key = 0.2, make_key(22)
    print(f"\npupo first step: T={r.T} N={r.N} width {r.N // cfg.num_minibatches}", flush=True)
    alg, state = run_gpu(r, cfg, params, device_recurrent_transition(tr, roll, extra), key, beta, max_steps=1)
    ex = alg.executor(state, r.T, r.N, r.obs_dim)
    flat = flat_state_of(state)
    g_gpu = leaves(tree_to_numpy(tree_from_flat(flat.program.layout, flat.G)))
    idx = ex.IDX.cpu().numpy()[:1]
    grads = []
    _, _, info = ppo.recurrent_pupo_update(to64(params), ppo.optimizer_init(to64(params)), plan,
                                           oracle_pupo_cfg(cfg), oracle_opt(r.optimizer), tr, key, beta,
                                           max_steps=1, indices=list(idx),
                                           record=lambda s, i, g, p: grads.append(g))
    far = info["margins"][0] > 1e-5
    assert far.mean() >= 0.99
    np.testing.assert_array_equal(idx[0][far], info["own_indices"][0][far])
    np.testing.assert_allclose(ex.WEIGHTS.cpu().numpy()[0], info["weights"][0], rtol=1e-4)
    for path, g in leaves(grads[0]).items():
        err = rel_l2(g_gpu[path], g)
        assert err <= 1e-4, (path, err)
    assert rel_l2(ex.RATIO.cpu().numpy(), info["ratio"]) <= 1e-4


def test_pupo_graph_replay_equals_eager():
    r, plan, params, tr, roll, extra = make_recurrent_case(4, T=8, N=64, M=4, E=2)
    cfg = pupo_cfg(r)
    out = []
    for use_graph in (False, True):
        alg, state = run_gpu(r, cfg, params, device_recurrent_transition(tr, roll, extra), make_key(23), 0.2,
                             use_graph=use_graph, updates=3)
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        out.append((flat_state_of(state).P.cpu().numpy().copy(), ex.RATIO.cpu().numpy().copy(),
                    ex.IDX.cpu().numpy().copy()))
    for a, b in zip(*out):
        np.testing.assert_array_equal(a, b)
