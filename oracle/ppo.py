"""Oracle PPO learner update (test infrastructure only; float64 throughout).

Restates, for the MLP and GRU actor-critics of the learner:

- ``loss_fn`` boonta/algorithms/ppo.py:77-146 and recurrent_ppo.py:101-184:
  ratio = exp(logp - old), approx KL, clip fraction, clipped surrogate,
  (clipped) value loss, entropy bonus; and its gradient as jax.value_and_grad
  takes it (ppo.py:155-157), including jax's tie rule for min/max (an equal
  pair shares the cotangent half and half) and jnp.clip = min(hi, max(lo, x)).
- the logged scalars ppo.py:167-180.
- ``optax.chain(clip_by_global_norm(m), adam(lr))`` of optax 0.2.8 (a
  third-party dependency, uv.lock:10743-10744; call sites
  hangar/recipes/ppo_cartpole.py:44-47, ppo.py:182-191): g <- g if
  ||g|| < m else (g / ||g||) * m; mu = (1-b1) g + b1 mu; nu = (1-b2) g^2 + b2 nu;
  count += 1; p <- p - lr * (mu / (1 - b1^count)) / (sqrt(nu / (1 - b2^count)) + eps).
- ``PPO.update`` ppo.py:199-233 and ``RecurrentPPO.update`` recurrent_ppo.py:186-281:
  bootstrap, GAE, optional normalisation, flatten (index t * N + n), split the
  key into E epoch keys, permute, reshape into M minibatches, scan.
- ``RecurrentPuPO.update`` recurrent_pupo.py:190-308: the same bootstrap; a
  ratio [N, T] of ones carried through E * M minibatch steps on the keys
  split(key, E * M); each step V-trace with rho = min(ratio, advantage_clip),
  c = min(ratio, trace_clip), prioritised env selection with replacement
  (oracle/priority.py), the minibatch advantages normalised and weighted per
  env, the recurrent loss, clip + Adam, and the step's ratios scattered back.
"""
from __future__ import annotations

import math

import numpy as np

from . import gae as _gae
from . import nets
from . import priority as _priority
from . import prng

FT = np.float64  # working precision (see nets.FT)


# ---------------------------------------------------------------- jax tie rule
def _d_min(x, y):
    """(d min(x,y)/dx, d min(x,y)/dy) with jax's balanced tie rule."""
    ans = np.minimum(x, y)
    ex, ey = (x == ans), (y == ans)
    dx = ex / np.where(ey, FT(2), FT(1))
    dy = ey / np.where(ex, FT(2), FT(1))
    return dx, dy


def _d_max(x, y):
    ans = np.maximum(x, y)
    ex, ey = (x == ans), (y == ans)
    dx = ex / np.where(ey, FT(2), FT(1))
    dy = ey / np.where(ex, FT(2), FT(1))
    return dx, dy


def _clip_and_grad(x, lo, hi):
    """jnp.clip(x, lo, hi) = minimum(hi, maximum(lo, x)) and d/dx."""
    m = np.maximum(lo, x)
    _, dm_dx = _d_max(np.full_like(x, lo), x)
    out = np.minimum(hi, m)
    _, dout_dm = _d_min(np.full_like(x, hi), m)
    return out, dout_dm * dm_dx


# ------------------------------------------------------------------- the loss
def loss_terms(logp, ent, value, old_logp, old_value, adv, ret, cfg):
    """Scalar loss, logs and the per-row cotangents (g_logp, g_ent, g_value)."""
    n = logp.shape[0]
    eps = cfg["clip_coefficient"]
    ratio = np.exp(logp - old_logp)
    kl = np.mean(old_logp - logp)
    clipfrac = np.mean((np.abs(ratio - 1.0) > eps).astype(FT))
    cr, dcr = _clip_and_grad(ratio, 1.0 - eps, 1.0 + eps)
    pg1, pg2 = ratio * adv, cr * adv
    actor = -np.minimum(pg1, pg2).mean()
    d1, d2 = _d_min(pg1, pg2)
    d_ratio = -(d1 * adv + d2 * adv * dcr) / n
    g_logp = d_ratio * ratio

    vl1 = 0.5 * (value - ret) ** 2
    if cfg["clip_value_loss"]:
        dv_clip, dcv = _clip_and_grad(value - old_value, -eps, eps)
        vc = old_value + dv_clip
        vl2 = 0.5 * (vc - ret) ** 2
        crit_rows = np.maximum(vl1, vl2)
        a1, a2 = _d_max(vl1, vl2)
        g_v_rows = a1 * (value - ret) + a2 * (vc - ret) * dcv
    else:
        crit_rows = vl1
        g_v_rows = value - ret
    critic = crit_rows.mean()
    entropy = ent.mean()
    loss = actor - cfg["entropy_coefficient"] * entropy + cfg["value_coefficient"] * critic
    g_value = cfg["value_coefficient"] * g_v_rows / n
    g_ent = np.full(n, -cfg["entropy_coefficient"] / n, FT)
    resid = ret - value
    logs = {
        "actor/loss": actor,
        "actor/entropy": entropy,
        "actor/approximate_kl": kl,
        "actor/clip_fraction": clipfrac,
        "actor/advantage": adv.mean(),
        "critic/loss": critic,
        "critic/explained_variance": 1.0 - resid.var() / (ret.var() + 1e-8),
        "critic/value": value.mean(),
    }
    return loss, logs, (g_logp, g_ent, g_value)


def _head_stats(params, plan, head, action):
    d = plan["dist"]
    if d["kind"] == "categorical":
        lp, ent, cache = nets.categorical_stats(head, action)
        return lp, ent, cache
    if d["kind"] == "gaussian":
        if d.get("scale") is not None:
            raw = np.broadcast_to(np.asarray(nets.get(params, d["scale"]), FT), head.shape)
            mean = head
        else:
            mean, raw = np.split(head, 2, axis=-1)
        sigma = nets.gaussian_sigma(raw)
        lp, ent = nets.gaussian_stats(mean, sigma, np.asarray(action, FT))
        return lp, ent, (mean, raw, sigma)
    raise ValueError(d["kind"])


def _head_grad(plan, cache, action, g_lp, g_ent, grads):
    d = plan["dist"]
    if d["kind"] == "categorical":
        return nets.categorical_grad(cache, action, g_lp, g_ent)
    mean, raw, sigma = cache
    dmean, dsig = nets.gaussian_grad(mean, sigma, np.asarray(action, FT), g_lp, g_ent)
    draw = dsig / (1.0 + np.exp(-raw))       # softplus' = sigmoid
    if d.get("scale") is not None:
        nets.add_in(grads, tuple(d["scale"]), draw.sum(0))
        return dmean
    return np.concatenate([dmean, draw], axis=-1)


def zeros_like_tree(t):
    if isinstance(t, dict):
        return {k: zeros_like_tree(v) for k, v in t.items()}
    return np.zeros(np.shape(t), FT)


def loss_and_grad(params, plan, cfg, obs, action, old_logp, old_value, adv, ret):
    """One minibatch of the MLP learner: loss, logs, grads (float64)."""
    head, value, cache = nets.forward(params, plan, obs)
    lp, ent, hcache = _head_stats(params, plan, head, action)
    loss, logs, (g_lp, g_ent, g_v) = loss_terms(
        lp, ent, value, np.asarray(old_logp, FT), np.asarray(old_value, FT),
        np.asarray(adv, FT), np.asarray(ret, FT), cfg)
    grads = zeros_like_tree(params)
    dhead = _head_grad(plan, hcache, action, g_lp, g_ent, grads)
    nets.backward(params, plan, cache, dhead, g_v, grads)
    return loss, logs, grads


def recurrent_loss_and_grad(params, plan, cfg, obs, done, carry, action, old_logp,
                            old_value, adv, ret, return_ratio=False):
    """One env-major sequence minibatch [B, T, ...] of RecurrentPPO.  With
    ``return_ratio`` also each sample's ratio exp(logp - old_logp) [B, T]
    (RecurrentPuPO's loss_fn returns it, recurrent_pupo.py:123,187)."""
    B, T = done.shape
    head, value, _, cache = nets.recurrent_forward(params, plan, obs, done, carry)
    hf = head.reshape(B * T, -1)
    act = np.asarray(action).reshape((B * T,) + np.shape(action)[2:])
    lp, ent, hcache = _head_stats(params, plan, hf, act)
    loss, logs, (g_lp, g_ent, g_v) = loss_terms(
        lp, ent, value.reshape(-1), np.asarray(old_logp, FT).reshape(-1),
        np.asarray(old_value, FT).reshape(-1), np.asarray(adv, FT).reshape(-1),
        np.asarray(ret, FT).reshape(-1), cfg)
    grads = zeros_like_tree(params)
    dhead = _head_grad(plan, hcache, act, g_lp, g_ent, grads)
    nets.recurrent_backward(params, plan, cache, dhead.reshape(B, T, -1),
                            g_v.reshape(B, T), grads)
    if return_ratio:
        return loss, logs, grads, np.exp(lp - np.asarray(old_logp, FT).reshape(-1)).reshape(B, T)
    return loss, logs, grads


# ------------------------------------------------------------------ optimizer
def tree_leaves(t, prefix=()):
    if isinstance(t, dict):
        out = []
        for k in sorted(t):
            out += tree_leaves(t[k], prefix + (k,))
        return out
    return [(prefix, t)]


def tree_map(f, *ts):
    if isinstance(ts[0], dict):
        return {k: tree_map(f, *(t[k] for t in ts)) for k in ts[0]}
    return f(*ts)


def optimizer_init(params):
    z = tree_map(lambda p: np.zeros(np.shape(p), FT), params)
    return {"count": 0, "mu": z, "nu": tree_map(np.copy, z)}


def optimizer_update(grads, state, params, opt):
    """clip_by_global_norm(max_grad_norm) then adam(lr, b1, b2, eps)."""
    gnorm = math.sqrt(sum(float((np.asarray(g, FT) ** 2).sum()) for _, g in tree_leaves(grads)))
    if opt.get("max_grad_norm") is not None and not gnorm < opt["max_grad_norm"]:
        grads = tree_map(lambda g: (g / gnorm) * opt["max_grad_norm"], grads)
    b1, b2, eps, lr = opt.get("b1", 0.9), opt.get("b2", 0.999), opt.get("eps", 1e-8), opt["lr"]
    count = state["count"] + 1
    mu = tree_map(lambda g, m: (1 - b1) * g + b1 * m, grads, state["mu"])
    nu = tree_map(lambda g, v: (1 - b2) * g * g + b2 * v, grads, state["nu"])
    c1, c2 = 1 - b1 ** count, 1 - b2 ** count
    new = tree_map(lambda p, m, v: np.asarray(p, FT) - lr * ((m / c1) / (np.sqrt(v / c2) + eps)),
                   params, mu, nu)
    return new, {"count": count, "mu": mu, "nu": nu}, gnorm


# ------------------------------------------------------------------- updates
def ppo_update(params, opt_state, plan, cfg, opt, tr, key, record=None, max_steps=None):
    """PPO.update (ppo.py:76-233) on a transition dict of [T, N, ...] arrays:
    obs (first.obs), next_obs_last (second.obs[-1]), action, reward,
    terminated, truncated, log_prob, value.  Returns (params, opt_state, logs).
    ``max_steps`` stops after that many minibatch steps (bootstrap, GAE and
    the permutations are whole)."""
    T, N = tr["reward"].shape
    B = T * N
    _, boot, _ = nets.forward(params, plan, tr["next_obs_last"])
    adv, ret = _gae.gae(tr["reward"], tr["terminated"], tr["truncated"], tr["value"],
                        boot, cfg["gamma"], cfg["gae_lambda"])
    if cfg.get("normalize_advantage"):
        adv = (adv - adv.mean()) / (adv.std() + 1e-8)
    flat = lambda a: np.asarray(a).reshape((B,) + np.shape(a)[2:])
    obs, act = flat(tr["obs"]), flat(tr["action"])
    olp, ov, fa, fr = flat(tr["log_prob"]), flat(tr["value"]), flat(adv), flat(ret)
    E, M = cfg["update_epochs"], cfg["num_minibatches"]
    perms = prng.epoch_permutations(key, E, B)
    logs = []
    steps = E * M if max_steps is None else min(max_steps, E * M)
    for step in range(steps):
        e, m = divmod(step, M)
        idx = perms[e].reshape(M, -1)[m]
        loss, lg, grads = loss_and_grad(params, plan, cfg, obs[idx], act[idx],
                                        olp[idx], ov[idx], fa[idx], fr[idx])
        params, opt_state, gnorm = optimizer_update(grads, opt_state, params, opt)
        lg["loss"] = loss
        lg["grad_norm"] = gnorm
        logs.append(lg)
        if record is not None:
            record(e, idx, grads, params)
    return params, opt_state, {"advantages": adv, "returns": ret, "bootstrap": boot,
                               "permutations": perms, "logs": logs}


def recurrent_ppo_update(params, opt_state, plan, cfg, opt, tr, key, record=None, max_steps=None):
    """RecurrentPPO.update (recurrent_ppo.py:98-281).  ``tr`` holds time-major
    [T, N, ...] obs, first_done (first.done), action, reward, terminated,
    truncated, log_prob, value, carry0 (carry[0], [N, H]), carry_last
    (carry[-1]), next_obs_last (second.obs[-1]) and next_done_last
    (second.done[-1])."""
    T, N = tr["reward"].shape
    # Transition.tail (utils/transition.py:20-26): a 2-step sequence of
    # (first[-1], second[-1]) from carry[-1]; the bootstrap is the 2nd value.
    seq_obs = np.stack([tr["obs"][-1], tr["next_obs_last"]], axis=1)
    seq_done = np.stack([tr["first_done"][-1], tr["next_done_last"]], axis=1)
    _, val, _, _ = nets.recurrent_forward(params, plan, seq_obs, seq_done, tr["carry_last"])
    boot = val[:, -1]
    adv, ret = _gae.gae(tr["reward"], tr["terminated"], tr["truncated"], tr["value"],
                        boot, cfg["gamma"], cfg["gae_lambda"])
    if cfg.get("normalize_advantage"):
        adv = (adv - adv.mean()) / (adv.std() + 1e-8)
    E, M = cfg["update_epochs"], cfg["num_minibatches"]
    perms = prng.epoch_permutations(key, E, N)
    em = lambda a, idx: np.moveaxis(np.take(np.asarray(a), idx, axis=1), 0, 1)
    logs = []
    steps = E * M if max_steps is None else min(max_steps, E * M)
    for step in range(steps):
        e, m = divmod(step, M)
        idx = perms[e].reshape(M, -1)[m]
        loss, lg, grads = recurrent_loss_and_grad(
            params, plan, cfg, em(tr["obs"], idx), em(tr["first_done"], idx),
            np.asarray(tr["carry0"])[idx], em(tr["action"], idx),
            em(tr["log_prob"], idx), em(tr["value"], idx), em(adv, idx), em(ret, idx))
        params, opt_state, gnorm = optimizer_update(grads, opt_state, params, opt)
        lg["loss"] = loss
        lg["grad_norm"] = gnorm
        logs.append(lg)
        if record is not None:
            record(e, idx, grads, params)
    return params, opt_state, {"advantages": adv, "returns": ret, "bootstrap": boot,
                               "permutations": perms, "logs": logs}


def recurrent_pupo_update(params, opt_state, plan, cfg, opt, tr, key, beta, record=None, max_steps=None,
                          indices=None):
    """RecurrentPuPO.update (recurrent_pupo.py:100-308) on the transition dict
    of ``recurrent_ppo_update``.  ``cfg`` adds advantage_clip, trace_clip,
    priority_exponent and normalize_advantage; ``beta`` is
    importance_exponent(state.step) (:208).  ``indices`` (a list of [width]
    arrays, one per step) replaces the oracle's own env draw at each step, so
    that a run whose advantages differ within rounding can be followed step by
    step; the oracle's own draws and their distances from a cumulative boundary
    are returned beside them."""
    T, N = tr["reward"].shape
    E, M = cfg["update_epochs"], cfg["num_minibatches"]
    width = N // M
    # bootstrap from the tail sequence (:193-203), as RecurrentPPO.update
    seq_obs = np.stack([tr["obs"][-1], tr["next_obs_last"]], axis=1)
    seq_done = np.stack([tr["first_done"][-1], tr["next_done_last"]], axis=1)
    _, val, _, _ = nets.recurrent_forward(params, plan, seq_obs, seq_done, tr["carry_last"])
    boot = val[:, -1]
    keys = prng.split(key, E * M)                      # :303-305
    ratio = np.ones((N, T), FT)                        # :306
    em = lambda a, idx: np.moveaxis(np.take(np.asarray(a), idx, axis=1), 0, 1)
    steps = E * M if max_steps is None else min(max_steps, E * M)
    info = {"bootstrap": boot, "indices": [], "weights": [], "own_indices": [], "margins": [],
            "probabilities": [], "logs": []}
    for step in range(steps):
        # V-trace on the carried ratio (:210-220, :226)
        rt = ratio.T
        adv, ret = _gae.gae(tr["reward"], tr["terminated"], tr["truncated"], tr["value"], boot,
                            cfg["gamma"], cfg["gae_lambda"], rho=np.minimum(rt, cfg["advantage_clip"]),
                            c=np.minimum(rt, cfg["trace_clip"]), dtype=FT)
        # prioritised selection with replacement (:228-236)
        own, _, prob, margin = _priority.priority_choice(adv, keys[step], width, cfg["priority_exponent"], beta)
        idx = own if indices is None else np.asarray(indices[step], np.int64)
        weight = (N * prob[idx]) ** (-float(beta))
        # env-major minibatch, normalised then weighted advantages (:238-253)
        scaled = em(adv, idx)
        if cfg.get("normalize_advantage", True):
            scaled = (scaled - scaled.mean()) / (scaled.std() + 1e-8)
        scaled = weight[:, None] * scaled
        loss, lg, grads, new_ratio = recurrent_loss_and_grad(
            params, plan, cfg, em(tr["obs"], idx), em(tr["first_done"], idx),
            np.asarray(tr["carry0"])[idx], em(tr["action"], idx), em(tr["log_prob"], idx),
            em(tr["value"], idx), scaled, em(ret, idx), return_ratio=True)
        params, opt_state, gnorm = optimizer_update(grads, opt_state, params, opt)
        lg["loss"] = loss
        lg["grad_norm"] = gnorm
        lg["actor/priority_weight"] = weight.mean()
        lg["actor/priority_beta"] = float(beta)
        info["logs"].append(lg)
        ratio[idx] = new_ratio                         # :297, stop_gradient
        for k, v in (("indices", idx), ("weights", weight), ("own_indices", own), ("margins", margin),
                     ("probabilities", prob)):
            info[k].append(v)
        if record is not None:
            record(step, idx, grads, params)
    info["advantages"], info["returns"], info["ratio"] = (adv, ret, ratio) if steps else (None, None, ratio)
    return params, opt_state, info
