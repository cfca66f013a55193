"""Seeded synthetic rollouts with the shapes and distributions of the five
learner workloads (numpy ``Generator(PCG64(seed))``, seed = 1000 + config):

  obs:    1, 3, 4: N(0, 1);  2: Bernoulli(0.1) in {0, 1};  5: per feature, 75 %
          Bernoulli(0.05) in {0, 1} and 25 % U(0, 1)
  reward: 1: 1.0;  2: Bernoulli(0.05);  3, 4: N(0, 1);  5: Bernoulli(0.02)
  done:   Bernoulli(p) -> terminated (truncated False, or with ``truncation``
          Bernoulli(p / 2) where not terminated); first.done[t] = second.done[t-1]
          and first.done[0] ~ Bernoulli(p) (same-step auto-reset order,
          boonta/environments/wrappers/same_step_auto_reset.py:12-27).

Observations come as one [T + 1, N, obs] array: first.obs = obs[:-1] and
second.obs = obs[1:].  Actions, log-probs and values are filled in by the caller
from the initial network, as a rollout would produce them.
"""
from __future__ import annotations

import numpy as np


def _obs(rng, name, shape):
    T1, N, D = shape
    if name == "discrete-anakin":
        return (rng.random(shape, dtype=np.float32) < 0.1).astype(np.float32)
    if name == "large-obs-bf16":
        binary = np.zeros(D, bool)
        binary[: (3 * D) // 4] = True
        rng.shuffle(binary)
        out = rng.random(shape, dtype=np.float32)
        out[..., binary] = (out[..., binary] < 0.05).astype(np.float32)
        return out
    return rng.standard_normal(shape, dtype=np.float32)


def _reward(rng, name, shape):
    if name == "discrete-tiny":
        return np.ones(shape, np.float32)
    if name == "discrete-anakin":
        return (rng.random(shape) < 0.05).astype(np.float32)
    if name == "large-obs-bf16":
        return (rng.random(shape) < 0.02).astype(np.float32)
    return rng.standard_normal(shape, dtype=np.float32)


def rollout(recipe, T: int | None = None, N: int | None = None, seed: int | None = None,
            truncation: bool = False) -> dict:
    T = T or recipe.T
    N = N or recipe.N
    rng = np.random.Generator(np.random.PCG64(recipe.seed if seed is None else seed))
    obs = _obs(rng, recipe.name, (T + 1, N, recipe.obs_dim))
    reward = _reward(rng, recipe.name, (T, N))
    p = recipe.done_p
    terminated = rng.random((T, N)) < p
    if truncation:
        truncated = (rng.random((T, N)) < p / 2) & ~terminated
    else:
        truncated = np.zeros((T, N), bool)
    done = terminated | truncated
    first_done = np.concatenate([rng.random((1, N)) < p, done[:-1]], axis=0)
    return {"obs": obs, "reward": reward, "terminated": terminated, "truncated": truncated,
            "first_done": first_done, "next_done_last": done[-1]}


def gumbel_max(rng, logits: np.ndarray) -> np.ndarray:
    """Categorical sample by the Gumbel-max trick (distributions.py:21-23)."""
    g = -np.log(-np.log(rng.random(logits.shape)))
    return np.argmax(logits + g, axis=-1).astype(np.int32)


def device_rollout(recipe, params, device, seed):
    """Seeded rollout of the workload's distributions generated on the device,
    with actions / log-probs / values from the initial network."""
    import torch
    import torch_ref
    from boonta_amd.types import Timestep, Transition

    T, N, D = recipe.T, recipe.N, recipe.obs_dim
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    shape = (T + 1, N, D)
    if recipe.name == "discrete-anakin":
        obs = (torch.rand(shape, device=device, generator=g) < 0.1).float()
    elif recipe.name == "large-obs-bf16":
        obs = torch.rand(shape, device=device, generator=g)
        binary = torch.zeros(D, dtype=torch.bool, device=device)
        binary[torch.randperm(D, device=device, generator=g)[: (3 * D) // 4]] = True
        obs[..., binary] = (obs[..., binary] < 0.05).float()
    else:
        obs = torch.randn(shape, device=device, generator=g)
    if recipe.name == "discrete-tiny":
        reward = torch.ones(T, N, device=device)
    elif recipe.name == "discrete-anakin":
        reward = (torch.rand(T, N, device=device, generator=g) < 0.05).float()
    elif recipe.name == "large-obs-bf16":
        reward = (torch.rand(T, N, device=device, generator=g) < 0.02).float()
    else:
        reward = torch.randn(T, N, device=device, generator=g)
    terminated = torch.rand(T, N, device=device, generator=g) < recipe.done_p
    truncated = torch.zeros(T, N, dtype=torch.bool, device=device)
    plan = recipe.network.plan(D)
    tparams = _to_torch(params, device)
    if plan["torso"] is not None:
        # first.done[t] = second.done[t-1] (same-step auto-reset); first.done[0] drawn
        first_term = torch.cat([torch.rand(1, N, device=device, generator=g) < recipe.done_p, terminated[:-1]])
        first_trunc = torch.zeros_like(first_term)
        H = plan["torso"]["features"]
        carry0 = torch.tanh(torch.randn(N, H, device=device, generator=g))
        action, logp, value, carry = torch_ref.recurrent_sample(tparams, plan, obs[:-1], first_term, carry0, g)
        return Transition(
            first=Timestep(obs=obs[:-1], terminated=first_term.contiguous(), truncated=first_trunc),
            second=Timestep(obs=obs[1:], action=action.contiguous(), reward=reward.contiguous(),
                            terminated=terminated, truncated=truncated),
            aux={"log_prob": logp.contiguous(), "value": value.contiguous()}, carry=carry.contiguous())
    acts, lps, vals = [], [], []
    flat_obs = obs[:-1].reshape(T * N, D)
    for s in range(0, T * N, 65536):
        a, lp, v = torch_ref.sample(tparams, plan, flat_obs[s:s + 65536], g)
        acts.append(a)
        lps.append(lp)
        vals.append(v)
    action = torch.cat(acts).reshape((T, N) + tuple(acts[0].shape[1:])).contiguous()
    tr = Transition(
        first=Timestep(obs=obs[:-1]),
        second=Timestep(obs=obs[1:], action=action, reward=reward.contiguous(), terminated=terminated,
                        truncated=truncated),
        aux={"log_prob": torch.cat(lps).reshape(T, N).contiguous(),
             "value": torch.cat(vals).reshape(T, N).contiguous()})
    return tr


def _to_torch(tree, device):
    import torch
    if isinstance(tree, dict):
        return {k: _to_torch(v, device) for k, v in tree.items()}
    return torch.from_numpy(np.asarray(tree, np.float32)).to(device)
