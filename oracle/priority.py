"""Oracle of RecurrentPuPO's prioritised env selection — TEST INFRASTRUCTURE ONLY.

Restates the minibatch selection of ``RecurrentPuPO.update``
(boonta/algorithms/recurrent_pupo.py:226-236):

    priority      = (sum over time of |advantages|) ** priority_exponent
    probabilities = (priority + 1e-6) / (priority.sum() + 1e-6)
    indices       = jax.random.choice(key, N, (width,), replace=True, p=probabilities)
    weight        = (N * probabilities[indices]) ** -beta

with jax 0.10.2's ``random.choice`` for ``replace=True`` and given ``p``
(jax/_src/random.py, third-party, absent here): the inverse CDF
``r = cumsum(p)[-1] * (1 - uniform(key, (width,)))``,
``indices = searchsorted(cumsum(p), r)`` (side 'left').  Uniform draws are
formed in float32 exactly as jax forms them (oracle/sample.py); everything
after them is float64.  Only ``tests/`` uses it.

Pinned by (tests/test_oracle_priority.py): the closed form of equal
priorities (index N - 1 - floor(N u), which a forward CDF draw or a 'right'
search would miss), a single-env distribution, a chi-square test of the draw
frequencies against ``probabilities``, the priority formula on a hand-computed
case, and the importance weights' closed form.  Parity with a live
``jax.random.choice`` stream: unpinned (jax absent).
"""
from __future__ import annotations

import numpy as np

from . import sample


def priorities(advantages, exponent: float) -> np.ndarray:
    """recurrent_pupo.py:228-231: |A| summed over time (axis 0 of the [T, N]
    V-trace output) raised to the priority exponent."""
    return np.abs(np.asarray(advantages, np.float64)).sum(axis=0) ** float(exponent)


def probabilities(advantages, exponent: float) -> np.ndarray:
    """recurrent_pupo.py:232."""
    pr = priorities(advantages, exponent)
    return (pr + 1e-6) / (pr.sum() + 1e-6)


def choice(key, p, width: int):
    """jax.random.choice(key, N, (width,), replace=True, p=p): inverse-CDF
    draws.  Returns (indices, margin): margin is each draw's distance from
    the nearest cumulative boundary relative to the total, where a float32
    cumulative sum taken in another order may pick the neighbouring index."""
    p = np.asarray(p, np.float64)
    c = np.cumsum(p)
    u = sample.uniform(key, width, 0.0, 1.0).astype(np.float64)
    r = c[-1] * (1.0 - u)
    idx = np.minimum(np.searchsorted(c, r, side="left"), len(p) - 1)
    lo = np.where(idx > 0, c[np.maximum(idx - 1, 0)], 0.0)
    margin = np.minimum(np.abs(r - c[idx]), np.abs(r - lo)) / c[-1]
    return idx.astype(np.int64), margin


def priority_choice(advantages, key, width: int, exponent: float, beta: float):
    """recurrent_pupo.py:226-236: (indices, weights, probabilities, margin)."""
    A = np.asarray(advantages)
    N = A.shape[1]
    prob = probabilities(A, exponent)
    idx, margin = choice(key, prob, width)
    weights = (N * prob[idx]) ** (-float(beta))
    return idx, weights, prob, margin


def choice_f32(key, p, width: int) -> np.ndarray:
    """jax.random.choice's inverse CDF taken the way jax types it: the
    cumulative sum of the float32 probabilities in float32 (here sequential,
    n in order; XLA may associate it otherwise) and r = c[-1] * (1 - u) in
    float32, then searchsorted (side 'left').  The product path draws on a
    float64 running sum instead; the two differ only for draws that fall
    between a float32 and a float64 cumulative boundary."""
    p = np.asarray(p, np.float32)
    c = np.cumsum(p, dtype=np.float32)
    u = sample.uniform(key, width, 0.0, 1.0).astype(np.float32)
    r = np.float32(c[-1]) * (np.float32(1.0) - u)
    idx = np.minimum(np.searchsorted(c, r, side="left"), len(p) - 1)
    return idx.astype(np.int64)
