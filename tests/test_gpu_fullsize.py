"""The first optimizer step of the learner at each workload's full size,
against the float64 oracle on the same inputs.

The whole-update tests run reduced shapes so that the oracle can replay every
step; the production launch shapes only run here: the discrete Anakin
workload's 32768-row minibatches (split-K weight gradients over 64 row
splits with their row-index caches, the fused head loss on 512 tiles), the
Gaussian workload's 2048-row towers on two streams, the GRU workload's
256 envs x 64 steps, and the large-observation bf16 workload's 8192 x 8268
first layer (bf16 observation copy, split-K forward, the 256 x 256 dW tile).
One step keeps the oracle at one minibatch (its bootstrap, GAE and
permutations are whole); both sides start from the same parameters, so the
bf16 step is teacher-forced by construction.

The rollout (observations, rewards, dones and the acting policy's actions,
log-probs and values) is generated on the GPU by the seeded synthetic
generator shared with the benchmark and copied to the host for the oracle.

Tolerances (written here): float32 workloads:
bootstrap, advantages and returns 1e-5 relative (atol 1e-5); the first
step's gradient and parameters 1e-4 relative (L2 per leaf); its logged
scalars 1e-5 relative (atol 1e-6).  bf16 workload: 2e-2 relative for the
bootstrap, advantages, returns, gradient and logs; the parameters after the
step against optax's clip + Adam restatement applied to the GPU's own
gradient, 1e-5 relative (atol 1e-8; Adam's first step moves each weight by
about lr whatever the size of its gradient, so an element whose bf16 gradient
rounds to the other side of zero steps the other way).  Permutations
bit-exact everywhere.
"""
import numpy as np
import pytest
import torch

import synthetic
from boonta_amd import recipes
from boonta_amd.algorithms.ppo import PPO, flat_state_of
from boonta_amd.algorithms.recurrent_ppo import RecurrentPPO
from boonta_amd.flat import tree_from_flat, tree_to_numpy
from boonta_amd.random import key as make_key
from oracle import ppo
from ppo_cases import oracle_cfg, oracle_opt, rel_l2, to64

pytestmark = pytest.mark.gpu


def host(t):
    return t.detach().cpu().numpy()


def oracle_transition(trans, recurrent: bool) -> dict:
    f, s, aux = trans.first, trans.second, trans.aux
    tr = {"obs": host(f.obs), "next_obs_last": host(s.obs[-1]), "action": host(s.action),
          "reward": host(s.reward), "terminated": host(s.terminated), "truncated": host(s.truncated),
          "log_prob": host(aux["log_prob"]), "value": host(aux["value"])}
    if recurrent:
        tr["first_done"] = host(f.terminated) | host(f.truncated)
        tr["carry0"] = host(trans.carry[0])
        tr["carry_last"] = host(trans.carry[-1])
        tr["next_done_last"] = tr["terminated"][-1] | tr["truncated"][-1]
    return tr


def leaves(tree):
    return dict(ppo.tree_leaves(tree))


@pytest.mark.parametrize("config", [2, 3, 4, 5])
def test_first_step_at_full_size(config):
    r = recipes.make(config)
    print(f"\nfull-size first step: workload {r.name} T={r.T} N={r.N} obs={r.obs_dim} "
          f"minibatch {r.minibatch}", flush=True)
    bf16 = r.network.plan(r.obs_dim)["compute_dtype"] == "bfloat16"
    tol = 2e-2 if bf16 else 1e-5
    gtol = 2e-2 if bf16 else 1e-4
    params = r.network.init(r.seed, r.obs_dim)["params"]
    trans = synthetic.device_rollout(r, params, torch.device("cuda:0"), r.seed)
    torch.cuda.synchronize()
    tr = oracle_transition(trans, r.recurrent)
    key = make_key(r.seed + 17)

    cls = RecurrentPPO if r.recurrent else PPO
    alg = cls(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=False)
    state = alg.init_from_params({"params": params}, r.obs_dim)
    ex = alg.executor(state, r.T, r.N, r.obs_dim)
    ex.KEY.copy_(torch.from_numpy(key.view(np.int32).copy()))
    ex.bind(alg._inputs(trans, r.obs_dim)[0])
    ex.issue(torch.cuda.current_stream().cuda_stream, max_steps=1)
    torch.cuda.synchronize()
    flat = flat_state_of(state)
    g_gpu = leaves(tree_to_numpy(tree_from_flat(flat.program.layout, flat.G)))
    p_gpu = leaves(tree_to_numpy(state.params["params"]))
    logs = alg.logs(state, r.T, r.N, r.obs_dim)
    boot, adv, ret, perm = host(ex.BOOT), host(ex.ADV), host(ex.RET), host(ex.PERM)
    del trans, alg, state, ex
    torch.cuda.empty_cache()

    grads = []
    update = ppo.recurrent_ppo_update if r.recurrent else ppo.ppo_update
    p_or, _, info = update(to64(params), ppo.optimizer_init(to64(params)), plan_of(r), oracle_cfg(r.cfg),
                           oracle_opt(r.optimizer), tr, key, max_steps=1,
                           record=lambda e, idx, g, p: grads.append(g))

    np.testing.assert_array_equal(perm, info["permutations"])
    if bf16:
        assert rel_l2(boot, info["bootstrap"]) <= tol
        assert rel_l2(adv, info["advantages"].reshape(-1)) <= tol
        assert rel_l2(ret, info["returns"].reshape(-1)) <= tol
    else:
        np.testing.assert_allclose(boot, info["bootstrap"], rtol=tol, atol=1e-5)
        np.testing.assert_allclose(adv, info["advantages"].reshape(-1), rtol=tol, atol=1e-5)
        np.testing.assert_allclose(ret, info["returns"].reshape(-1), rtol=tol, atol=1e-5)
    worst_g = 0.0
    for path, g in leaves(grads[0]).items():
        err = rel_l2(g_gpu[path], g)
        worst_g = max(worst_g, err)
        assert err <= gtol, (path, err)
    worst_p = 0.0
    if bf16:
        # an element whose bf16 gradient rounds to the other side of zero takes
        # Adam's opposite lr step: the GPU's clip + Adam step on its own
        # gradient against optax's restatement (1e-5 relative, 1e-8 absolute)
        p_or, _, _ = ppo.optimizer_update(tree_of(g_gpu), ppo.optimizer_init(to64(params)), to64(params),
                                          oracle_opt(r.optimizer))
        for path, p in leaves(p_or).items():
            np.testing.assert_allclose(p_gpu[path], p, rtol=1e-5, atol=1e-8, err_msg=str(path))
    for path, p in leaves(p_or).items():
        err = rel_l2(p_gpu[path], p)
        worst_p = max(worst_p, err)
        assert err <= 1e-4, (path, err)
    for k, v in info["logs"][0].items():
        if k == "grad_norm":
            continue
        if bf16:
            np.testing.assert_allclose(logs[k][0], v, rtol=tol, atol=1e-3, err_msg=k)
        else:
            np.testing.assert_allclose(logs[k][0], v, rtol=1e-5, atol=1e-6, err_msg=k)
    print(f"{r.name}: worst gradient rel-L2 {worst_g:.2e}, parameters {worst_p:.2e}", flush=True)


def plan_of(recipe):
    return recipe.network.plan(recipe.obs_dim)


def tree_of(flat_leaves):
    out = {}
    for path, v in flat_leaves.items():
        node = out
        for key in path[:-1]:
            node = node.setdefault(key, {})
        node[path[-1]] = np.asarray(v, np.float64)
    return out
