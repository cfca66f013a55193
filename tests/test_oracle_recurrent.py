"""Pins the oracle's RecurrentPPO.update restatement with the reference's own
recurrent invariants (no GPU):

- the first minibatch step replays exactly the log-probs the rollout acted on
  (tests/test_algorithms.py:398-408): ratio 1, approximate KL 0, clip
  fraction 0 on every sequence minibatch of the first step;
- the tail bootstrap (Transition.tail, utils/transition.py:20-26) equals the
  value the next step would see when the rollout forward runs one step
  further (tests/test_algorithms.py:510-535);
- an episode start forgets the past (tests/test_networks.py:60-66).
"""
import numpy as np

from oracle import nets, ppo
from ppo_cases import make_recurrent_case, oracle_cfg, oracle_opt, to64
from boonta_amd.random import key as make_key


def test_first_step_replays_the_rollout_log_probs():
    r, plan, params, tr, roll, extra = make_recurrent_case(4, T=6, N=16, M=2, E=1)
    _, _, info = ppo.recurrent_ppo_update(to64(params), ppo.optimizer_init(to64(params)), plan,
                                          oracle_cfg(r.cfg), oracle_opt(r.optimizer), tr, make_key(3))
    first = info["logs"][0]
    # the stored log-probs are float32: the replay matches to their rounding (the reference test: atol 1e-5)
    assert abs(first["actor/approximate_kl"]) < 1e-6
    assert first["actor/clip_fraction"] == 0.0


def test_tail_bootstrap_is_the_next_steps_value():
    r, plan, params, tr, roll, extra = make_recurrent_case(4, T=5, N=8, M=2, E=1)
    T, N = tr["reward"].shape
    _, _, info = ppo.recurrent_ppo_update(to64(params), ppo.optimizer_init(to64(params)), plan,
                                          oracle_cfg(r.cfg), oracle_opt(r.optimizer), tr, make_key(0))
    # the same network run over T + 1 steps from carry[0]; its last value is the bootstrap
    obs = np.concatenate([tr["obs"], tr["next_obs_last"][None]], axis=0)
    done = np.concatenate([tr["first_done"], tr["next_done_last"][None]], axis=0)
    _, value, _, _ = nets.recurrent_forward(to64(params), plan, np.moveaxis(obs, 0, 1), done.T, tr["carry0"])
    np.testing.assert_allclose(info["bootstrap"], value[:, -1], rtol=1e-6, atol=1e-6)


def test_an_episode_start_forgets_the_past():
    r, plan, params, tr, roll, extra = make_recurrent_case(4, T=4, N=8, M=2, E=1)
    obs = np.moveaxis(tr["obs"], 0, 1)
    done = np.zeros((8, 4), bool)
    done[:, 2] = True
    rng = np.random.default_rng(5)
    c1, c2 = rng.standard_normal((2, 8, plan["torso"]["features"]))
    o1 = obs.copy()
    o2 = obs.copy()
    o2[:, :2] = rng.standard_normal(o2[:, :2].shape)
    h1, v1, _, _ = nets.recurrent_forward(to64(params), plan, o1, done, c1)
    h2, v2, _, _ = nets.recurrent_forward(to64(params), plan, o2, done, c2)
    np.testing.assert_allclose(h1[:, 2:], h2[:, 2:], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(v1[:, 2:], v2[:, 2:], rtol=1e-12, atol=1e-12)
    assert not np.allclose(v1[:, :2], v2[:, :2])
