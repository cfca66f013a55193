"""Oracle of the rollout-side action sampling — TEST INFRASTRUCTURE ONLY.

Restates ``dist.sample_and_log_prob(seed=key)`` as boonta's ``PPO.step`` calls
it (boonta/algorithms/ppo.py:57-74) for the categorical head
(boonta/networks/distributions.py:8-23, distrax 0.1.9 ``Categorical``) and the
diagonal Gaussian head (distributions.py:42-57, distrax
``MultivariateNormalDiag``), with jax 0.10.2's ``random.uniform`` /
``random.gumbel`` / ``random.normal`` on the partitionable Threefry stream.
Uniform draws are formed in float32 exactly as jax forms them; everything after
them is float64.  Only ``tests/``, ``bench.py``'s CPU baseline and
``__graft_entry__.smoke`` use it.

Pinned by (tests/test_oracle_sample.py): hand-computed words -> uniform
endpoints; chi-square of Gumbel-max frequencies against softmax
probabilities; moments and a Kolmogorov-Smirnov test of the normal draws;
sqrt(2) erfinv(u) against the normal quantile function; log-probs against
scipy's Normal log-density and log-softmax; the greedy (temperature 0) case.
Parity with a live ``jax.random`` bit stream: unpinned (jax absent).
"""
from __future__ import annotations

import numpy as np
from scipy import special

from . import prng

F32 = np.float32
TINY32 = np.finfo(np.float32).tiny
NEXT_ABOVE_MINUS_ONE = np.nextafter(F32(-1.0), F32(0.0), dtype=F32)


def uniform(key, n: int, minval, maxval) -> np.ndarray:
    """jax.random.uniform(key, (n,), float32, minval, maxval): the top 23 bits
    of each 32-bit word as the mantissa of a float in [1, 2), minus 1, times
    (maxval - minval) rounded to float32, plus minval, floored at minval."""
    return words_to_uniform(prng.random_bits32(key, n), minval, maxval)


def words_to_uniform(bits, minval, maxval) -> np.ndarray:
    """The float32 arithmetic of jax.random.uniform on given 32-bit words."""
    bits = np.asarray(bits, np.uint32)
    f = ((bits >> np.uint32(9)) | np.uint32(0x3F800000)).view(F32) - F32(1.0)
    lo, hi = F32(minval), F32(maxval)
    span = F32(hi - lo)
    return np.maximum(lo, F32(f * span) + lo)


def gumbel(key, n: int) -> np.ndarray:
    """jax.random.gumbel, low-dynamic-range form: -log(-log(u)), u ~ U[tiny, 1)."""
    u = uniform(key, n, TINY32, 1.0).astype(np.float64)
    return -np.log(-np.log(u))


def normal(key, n: int) -> np.ndarray:
    """jax.random.normal: sqrt(2) erfinv(u), u ~ U[nextafter(-1, 0), 1)."""
    u = uniform(key, n, NEXT_ABOVE_MINUS_ONE, 1.0).astype(np.float64)
    return np.sqrt(2.0) * special.erfinv(u)


def log_softmax(x: np.ndarray) -> np.ndarray:
    m = np.max(x, axis=-1, keepdims=True)
    s = x - m
    return s - np.log(np.sum(np.exp(s), axis=-1, keepdims=True))


def categorical_sample(preferences, key, temperature: float = 1.0):
    """Returns (action int32 [rows], log_prob [rows], margin [rows]): the
    Gumbel-max draw of Categorical(preferences, temperature)
    (distributions.py:9-23), its log-probability, and the gap between the
    two largest perturbed logits (how close the draw was to a tie)."""
    pref = np.asarray(preferences, np.float64)
    rows, A = pref.shape
    if temperature > 0:
        logits = log_softmax(pref / temperature)
    else:
        greedy = np.argmax(log_softmax(pref), axis=-1)
        logits = np.full_like(pref, -np.inf)
        logits[np.arange(rows), greedy] = 0.0
    z = logits + gumbel(key, rows * A).reshape(rows, A)
    action = np.argmax(z, axis=-1).astype(np.int32)
    if A > 1:
        top2 = np.sort(z, axis=-1)[:, -2:]
        margin = top2[:, 1] - top2[:, 0]
    else:
        margin = np.full(rows, np.inf)
    return action, logits[np.arange(rows), action], margin


def softplus(x):
    x = np.asarray(x, np.float64)
    return np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))


def gaussian_sample(mean, raw_scale, key, temperature: float = 1.0):
    """Returns (action [rows, D], log_prob [rows], eps [rows, D]) of
    MultivariateNormalDiag(mean, temperature * (softplus(s) + 1e-3))
    sampled through distrax's bijector form: eps ~ N(0, 1), action =
    sigma * eps + mean, log_prob = sum(-eps^2 / 2 - log(2 pi) / 2) - sum(log sigma)."""
    mean = np.asarray(mean, np.float64)
    rows, D = mean.shape
    sigma = temperature * (softplus(np.broadcast_to(raw_scale, mean.shape)) + 1e-3)
    eps = normal(key, rows * D).reshape(rows, D)
    action = sigma * eps + mean
    lp = np.sum(-0.5 * eps * eps - 0.5 * np.log(2 * np.pi), axis=-1) - np.sum(np.log(sigma), axis=-1)
    return action, lp, eps
