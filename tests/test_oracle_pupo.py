"""Pins the oracle's RecurrentPuPO.update (oracle/ppo.py recurrent_pupo_update,
boonta/algorithms/recurrent_pupo.py:100-308) by reductions to already pinned
pieces: one step with unit clips, beta 0 and no normalisation is a
RecurrentPPO step on plain GAE advantages of the drawn envs; the ratio a step
scatters back is exp(logp - old_logp) of an independent forward on the drawn
envs, it stays 1 elsewhere, and the next step's V-trace runs on it; with beta
0 the normalised minibatch advantages have mean 0."""
import numpy as np
import pytest

from oracle import gae as ogae
from oracle import nets, ppo, prng
from oracle import priority as opriority
from ppo_cases import make_recurrent_case, oracle_cfg, oracle_opt, to64


def pupo_cfg(r, **kw):
    cfg = oracle_cfg(r.cfg)
    cfg.update(advantage_clip=1.0, trace_clip=1.0, priority_exponent=0.8, normalize_advantage=True)
    cfg.update(kw)
    return cfg


def case(seed=0, off_policy=False):
    r, plan, params, tr, roll, extra = make_recurrent_case(4, T=6, N=16, M=4, E=2, seed=seed)
    if off_policy:
        # log-probs of another policy: ratios away from 1
        rng = np.random.default_rng(seed + 5)
        tr = dict(tr, log_prob=(tr["log_prob"] + rng.normal(0, 0.3, tr["log_prob"].shape)).astype(np.float32))
    return r, plan, to64(params), tr


def test_one_step_reduces_to_recurrent_ppo_on_gae():
    r, plan, params, tr = case()
    cfg = pupo_cfg(r, normalize_advantage=False)
    grads = []
    key = prng.key(3)
    _, _, info = ppo.recurrent_pupo_update(params, ppo.optimizer_init(params), plan, cfg, oracle_opt(r.optimizer),
                                           tr, key, beta=0.0, max_steps=1,
                                           record=lambda s, idx, g, p: grads.append(g))
    idx = info["indices"][0]
    np.testing.assert_array_equal(info["weights"][0], 1.0)
    # plain GAE (ratio 1, unit clips) and the recurrent loss on the drawn envs
    adv, ret = ogae.gae(tr["reward"], tr["terminated"], tr["truncated"], tr["value"], info["bootstrap"],
                        cfg["gamma"], cfg["gae_lambda"])
    em = lambda a: np.moveaxis(np.take(np.asarray(a), idx, axis=1), 0, 1)
    _, _, want = ppo.recurrent_loss_and_grad(params, plan, cfg, em(tr["obs"]), em(tr["first_done"]),
                                             np.asarray(tr["carry0"])[idx], em(tr["action"]), em(tr["log_prob"]),
                                             em(tr["value"]), em(adv), em(ret))
    for path, g in ppo.tree_leaves(want):
        np.testing.assert_allclose(dict(ppo.tree_leaves(grads[0]))[path], g, rtol=1e-12, atol=1e-14)
    # the draw is jax.random.choice on the first of split(key, E * M)
    k0 = prng.split(key, r.cfg.update_epochs * r.cfg.num_minibatches)[0]
    own, _, _, _ = opriority.priority_choice(adv, k0, len(idx), 0.8, 0.0)
    np.testing.assert_array_equal(idx, own)


def test_scattered_ratio_feeds_the_next_vtrace():
    r, plan, params, tr = case(seed=1, off_policy=True)
    cfg = pupo_cfg(r, advantage_clip=1.1, trace_clip=0.9)
    _, _, info = ppo.recurrent_pupo_update(params, ppo.optimizer_init(params), plan, cfg, oracle_opt(r.optimizer),
                                           tr, prng.key(4), beta=0.4, max_steps=2)
    idx = info["indices"][0]
    # exp(logp - old_logp) of the initial parameters on the drawn envs, from an independent forward
    obs_em = np.moveaxis(tr["obs"], 0, 1)[idx]
    head, _, _, _ = nets.recurrent_forward(params, plan, obs_em, tr["first_done"].T[idx], tr["carry0"][idx])
    act = tr["action"].T[idx]
    lp, _, _ = nets.categorical_stats(head.reshape(-1, head.shape[-1]), act.reshape(-1))
    want = np.ones((tr["reward"].shape[1], tr["reward"].shape[0]))
    want[idx] = np.exp(lp.reshape(act.shape) - tr["log_prob"].T[idx])
    assert np.abs(want - 1.0).max() > 0.05        # the case is off-policy
    # step 2's V-trace ran on that ratio (its scatter of step 2 is the final ratio)
    rt = want.T
    adv2, _ = ogae.gae(tr["reward"], tr["terminated"], tr["truncated"], tr["value"], info["bootstrap"],
                       cfg["gamma"], cfg["gae_lambda"], rho=np.minimum(rt, 1.1), c=np.minimum(rt, 0.9))
    np.testing.assert_allclose(info["advantages"], adv2, rtol=1e-12, atol=1e-14)
    untouched = np.setdiff1d(np.arange(len(want)), np.concatenate(info["indices"]))
    np.testing.assert_array_equal(info["ratio"][untouched], 1.0)


@pytest.mark.parametrize("normalize", [True, False])
def test_beta_zero_logs_and_weights(normalize):
    r, plan, params, tr = case(seed=2)
    cfg = pupo_cfg(r, normalize_advantage=normalize)
    _, _, info = ppo.recurrent_pupo_update(params, ppo.optimizer_init(params), plan, cfg, oracle_opt(r.optimizer),
                                           tr, prng.key(5), beta=0.0, max_steps=3)
    for lg, w in zip(info["logs"], info["weights"]):
        np.testing.assert_array_equal(w, 1.0)
        assert lg["actor/priority_weight"] == 1.0 and lg["actor/priority_beta"] == 0.0
        if normalize:
            assert abs(lg["actor/advantage"]) < 1e-12
    # beta 1: (N p)^-1 weights, their mean under the draw is about one
    _, _, info = ppo.recurrent_pupo_update(params, ppo.optimizer_init(params), plan, cfg, oracle_opt(r.optimizer),
                                           tr, prng.key(5), beta=1.0, max_steps=1)
    p, idx, w = info["probabilities"][0], info["indices"][0], info["weights"][0]
    np.testing.assert_allclose(w, 1.0 / (len(p) * p[idx]), rtol=1e-12)
