"""Whole-update parity of the HIP learner against the float64 oracle on the
same seeded inputs (configs at sizes the oracle finishes in seconds), plus
graph == eager and run-to-run determinism.

Tolerances (written here): advantages / returns 1e-5
relative (atol 1e-6); permutations bit-exact; the first minibatch gradient
and the parameters after the update 1e-4 relative (L2 per leaf); the logged
losses of every minibatch step 1e-5 relative plus an absolute floor of 1e-6
for quantities that cross zero."""
import numpy as np
import pytest
import torch

from boonta_amd.flat import tree_from_flat, tree_to_numpy
from boonta_amd.algorithms.ppo import flat_state_of
from boonta_amd.random import key as make_key
from oracle import ppo
from ppo_cases import device_transition, gpu_algorithm, make_case, oracle_cfg, oracle_opt, rel_l2, to64

pytestmark = pytest.mark.gpu

CASES = {
    "c1-full": dict(config=1),
    "c2-small": dict(config=2, T=16, N=64, M=4, E=2),
    "c3-small": dict(config=3, T=8, N=64, M=4, E=2),
}


def run_both(case, key_seed=42, truncation=False, max_steps=None):
    r, plan, params, tr, roll = make_case(**case, truncation=truncation)
    key = make_key(key_seed)
    records = []
    p_or, s_or, info = ppo.ppo_update(to64(params), ppo.optimizer_init(to64(params)), plan, oracle_cfg(r.cfg),
                                      oracle_opt(r.optimizer), tr, key,
                                      record=lambda e, idx, g, p: records.append((idx.copy(), g)))
    alg = gpu_algorithm(r, use_graph=False)
    state = alg.init_from_params({"params": params}, r.obs_dim)
    trans = device_transition(tr, roll)
    if max_steps is None:
        alg.update(state, key, trans)
    else:
        ex = alg.executor(state, r.T, r.N, r.obs_dim)
        ex.KEY.copy_(torch.from_numpy(key.view(np.int32).copy()))
        ex.bind(alg._inputs(trans, r.obs_dim)[0])
        ex.issue(torch.cuda.current_stream().cuda_stream, max_steps=max_steps)
    torch.cuda.synchronize()
    return r, alg, state, (p_or, s_or, info, records)


def leaves(tree):
    return dict(ppo.tree_leaves(tree))


@pytest.mark.parametrize("name", list(CASES))
def test_advantages_returns_and_permutations(name):
    r, alg, state, (p_or, s_or, info, _) = run_both(CASES[name], truncation=True)
    ex = alg.executor(state, r.T, r.N, r.obs_dim)
    np.testing.assert_allclose(ex.ADV.cpu().numpy(), info["advantages"].reshape(-1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ex.RET.cpu().numpy(), info["returns"].reshape(-1), rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(ex.PERM.cpu().numpy(), info["permutations"])
    np.testing.assert_allclose(ex.BOOT.cpu().numpy(), info["bootstrap"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name", list(CASES))
def test_first_minibatch_gradient(name):
    r, alg, state, (_, _, _, records) = run_both(CASES[name], max_steps=1)
    flat = flat_state_of(state)
    g_gpu = leaves(tree_to_numpy(tree_from_flat(flat.program.layout, flat.G)))
    g_or = leaves(records[0][1])
    assert set(g_gpu) == set(g_or)
    for path, g in g_or.items():
        err = rel_l2(g_gpu[path], g)
        assert err <= 1e-4, (path, err)


@pytest.mark.parametrize("name", list(CASES))
def test_parameters_and_logs_after_the_update(name):
    r, alg, state, (p_or, s_or, info, _) = run_both(CASES[name])
    p_gpu = leaves(tree_to_numpy(state.params["params"]))
    worst = 0.0
    for path, p in leaves(p_or).items():
        err = rel_l2(p_gpu[path], p)
        worst = max(worst, err)
        assert err <= 1e-4, (path, err)
    assert int(flat_state_of(state).count.item()) == r.cfg.update_epochs * r.cfg.num_minibatches
    logs = alg.logs(state, r.T, r.N, r.obs_dim)
    for i, lg in enumerate(info["logs"]):
        for k, v in lg.items():
            if k == "grad_norm":
                continue
            np.testing.assert_allclose(logs[k][i], v, rtol=1e-5, atol=1e-6, err_msg=f"step {i} {k}")
    print(f"{name}: worst parameter rel-L2 {worst:.2e}")


@pytest.mark.parametrize("name", ["c2-small", "c3-small"])
def test_graph_replay_equals_eager_and_is_deterministic(name):
    """Shared trunk, and separate actor/critic towers (whose chains run on two
    streams, forked and joined inside the captured graph)."""
    case = CASES[name]
    results = []
    for use_graph in (False, True, True):
        r, plan, params, tr, roll = make_case(**case)
        alg = gpu_algorithm(r, use_graph=use_graph)
        state = alg.init_from_params({"params": params}, r.obs_dim)
        trans = device_transition(tr, roll)
        for k in (1, 2, 3):   # three updates: the graph is captured once and replayed
            alg.update(state, make_key(k), trans)
        torch.cuda.synchronize()
        results.append(flat_state_of(state).P.cpu().numpy().copy())
    np.testing.assert_array_equal(results[0], results[1])
    np.testing.assert_array_equal(results[1], results[2])


@pytest.mark.parametrize("recurrent", [False, True])
def test_fresh_rollout_buffers_reuse_one_graph_and_equal_eager(recurrent):
    """A caller that hands in a different rollout buffer every update (two
    buffers alternating, then one written into rollout_buffers): the graph
    path copies each into the executor's own buffers and replays the one
    graph it captured, bit-identical to the eager path on the same sequence."""
    from ppo_cases import device_recurrent_transition, gpu_recurrent_algorithm, make_recurrent_case
    if recurrent:
        cases = [make_recurrent_case(4, T=8, N=64, M=4, E=2, seed=s) for s in (0, 1)]
        r, params = cases[0][0], cases[0][2]
        rollouts = [device_recurrent_transition(c[3], c[4], c[5]) for c in cases]
        make_alg = lambda g: gpu_recurrent_algorithm(r, use_graph=g)
    else:
        cases = [make_case(config=2, T=16, N=64, M=4, E=2, seed=s) for s in (0, 1)]
        r, params = cases[0][0], cases[0][2]
        rollouts = [device_transition(c[3], c[4]) for c in cases]
        make_alg = lambda g: gpu_algorithm(r, use_graph=g)
    results = []
    for use_graph in (False, True):
        alg = make_alg(use_graph)
        state = alg.init_from_params({"params": params}, r.obs_dim)
        for k, tr in enumerate([rollouts[0], rollouts[1], rollouts[0], rollouts[1]]):
            alg.update(state, make_key(10 + k), tr)
        own = alg.rollout_buffers(state, r.T, r.N, r.obs_dim, fill_from=rollouts[0])
        alg.update(state, make_key(20), own)
        torch.cuda.synchronize()
        results.append(flat_state_of(state).P.cpu().numpy().copy())
        if use_graph:
            assert len(alg.executor(state, r.T, r.N, r.obs_dim).graphs) == 1
    np.testing.assert_array_equal(results[0], results[1])
