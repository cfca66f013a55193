"""Shared builders for the learner parity tests: a seeded synthetic rollout
whose actions, log-probs and values come from the initial network (computed by
the oracle in float64), fed identically to the oracle and to the HIP path."""
from __future__ import annotations

import numpy as np
import torch

import synthetic
from boonta_amd import recipes
from boonta_amd.algorithms.ppo import PPO
from boonta_amd.types import Timestep, Transition
from oracle import nets, ppo


def oracle_cfg(cfg) -> dict:
    return {"clip_coefficient": cfg.clip_coefficient, "clip_value_loss": cfg.clip_value_loss,
            "entropy_coefficient": cfg.entropy_coefficient, "value_coefficient": cfg.value_coefficient,
            "gamma": cfg.gamma, "gae_lambda": cfg.gae_lambda, "update_epochs": cfg.update_epochs,
            "num_minibatches": cfg.num_minibatches, "normalize_advantage": cfg.normalize_advantage}


def oracle_opt(chain) -> dict:
    a = chain.adam
    return {"lr": a.learning_rate, "b1": a.b1, "b2": a.b2, "eps": a.eps, "max_grad_norm": chain.max_grad_norm}


def to64(tree):
    return ppo.tree_map(lambda a: np.asarray(a, np.float64), tree)


def make_case(config: int, T=None, N=None, M=None, E=None, seed=0, truncation=False):
    r = recipes.make(config).resized(T=T, N=N, num_minibatches=M, update_epochs=E)
    T, N, D = r.T, r.N, r.obs_dim
    roll = synthetic.rollout(r, T, N, truncation=truncation)
    plan = r.network.plan(D)
    params = r.network.init(seed, D)["params"]
    rng = np.random.default_rng(seed + 77)
    first = roll["obs"][:-1]
    head, value, _ = nets.forward(params, plan, first.reshape(T * N, D))
    d = plan["dist"]
    if d["kind"] == "categorical":
        action = synthetic.gumbel_max(rng, head).reshape(T, N)
        lp, _, _ = nets.categorical_stats(head, action.reshape(-1))
    else:
        Dm = d["dim"]
        if d.get("scale") is not None:
            raw = np.broadcast_to(np.asarray(nets.get(params, d["scale"]), np.float64), head.shape)
            mean = head
        else:
            mean, raw = head[:, :Dm], head[:, Dm:]
        sig = nets.gaussian_sigma(raw)
        a = mean + sig * rng.standard_normal(mean.shape)
        action = a.astype(np.float32).reshape(T, N, Dm)
        lp, _ = nets.gaussian_stats(mean, sig, action.reshape(T * N, Dm).astype(np.float64))
    tr = {
        "obs": first, "next_obs_last": roll["obs"][-1], "action": action, "reward": roll["reward"],
        "terminated": roll["terminated"], "truncated": roll["truncated"],
        "log_prob": lp.astype(np.float32).reshape(T, N), "value": value.astype(np.float32).reshape(T, N),
    }
    return r, plan, params, tr, roll


def device_transition(tr, roll, device="cuda") -> Transition:
    obs = torch.from_numpy(roll["obs"]).to(device)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    first = Timestep(obs=obs[:-1])
    second = Timestep(obs=obs[1:], action=f(tr["action"]), reward=f(tr["reward"]),
                      terminated=f(tr["terminated"]), truncated=f(tr["truncated"]))
    return Transition(first=first, second=second, aux={"log_prob": f(tr["log_prob"]), "value": f(tr["value"])})


def gpu_algorithm(r, use_graph=True) -> PPO:
    return PPO(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def make_recurrent_case(config: int = 4, T=None, N=None, M=None, E=None, seed=0, truncation=False):
    """A seeded recurrent rollout: actions, log-probs and values from the
    initial network run over the whole rollout (env-major, from carry[0], with
    the resets first.done), and carry[-1] = the carry entering the last step,
    as Anakin.rollout records them (podracers/anakin.py:46-76)."""
    r = recipes.make(config).resized(T=T, N=N, num_minibatches=M, update_epochs=E)
    T, N, D = r.T, r.N, r.obs_dim
    roll = synthetic.rollout(r, T, N, truncation=truncation)
    plan = r.network.plan(D)
    H = plan["torso"]["features"]
    params = r.network.init(seed, D)["params"]
    rng = np.random.default_rng(seed + 91)
    first_term = np.concatenate([roll["first_done"][:1], roll["terminated"][:-1]], axis=0)
    first_trunc = np.concatenate([np.zeros((1, N), bool), roll["truncated"][:-1]], axis=0)
    first_done = first_term | first_trunc
    carry0 = np.tanh(rng.standard_normal((N, H))).astype(np.float32)
    obs_em = np.moveaxis(roll["obs"][:-1], 0, 1)
    head, value, _, _ = nets.recurrent_forward(params, plan, obs_em, first_done.T, carry0)
    if T > 1:
        _, _, carry_last, _ = nets.recurrent_forward(params, plan, obs_em[:, :T - 1], first_done.T[:, :T - 1],
                                                     carry0)
    else:
        carry_last = carry0
    carry_last = np.asarray(carry_last, np.float32)
    logits = np.moveaxis(head, 0, 1).reshape(T * N, -1)
    action = synthetic.gumbel_max(rng, logits).reshape(T, N)
    lp, _, _ = nets.categorical_stats(logits, action.reshape(-1))
    tr = {
        "obs": roll["obs"][:-1], "first_done": first_done, "action": action, "reward": roll["reward"],
        "terminated": roll["terminated"], "truncated": roll["truncated"],
        "log_prob": lp.astype(np.float32).reshape(T, N), "value": np.moveaxis(value, 0, 1).astype(np.float32),
        "carry0": carry0, "carry_last": carry_last, "next_obs_last": roll["obs"][-1],
        "next_done_last": roll["terminated"][-1] | roll["truncated"][-1],
    }
    carry = np.zeros((T, N, H), np.float32)
    carry[0] = carry0
    carry[-1] = carry_last
    extra = {"first_terminated": first_term, "first_truncated": first_trunc, "carry": carry}
    return r, plan, params, tr, roll, extra


def device_recurrent_transition(tr, roll, extra, device="cuda") -> Transition:
    obs = torch.from_numpy(roll["obs"]).to(device)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    first = Timestep(obs=obs[:-1], terminated=f(extra["first_terminated"]), truncated=f(extra["first_truncated"]))
    second = Timestep(obs=obs[1:], action=f(tr["action"]), reward=f(tr["reward"]),
                      terminated=f(tr["terminated"]), truncated=f(tr["truncated"]))
    return Transition(first=first, second=second, aux={"log_prob": f(tr["log_prob"]), "value": f(tr["value"])},
                      carry=f(extra["carry"]))


def gpu_recurrent_algorithm(r, use_graph=True):
    from boonta_amd.algorithms.recurrent_ppo import RecurrentPPO
    return RecurrentPPO(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=use_graph)
