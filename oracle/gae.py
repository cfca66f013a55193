"""Oracle GAE (test infrastructure only).

Restates boonta/algorithms/advantage_estimators.py:8-56
(``generalized_advantage_estimator``): a reverse scan over time with the carry
``(advantage, next_value)`` initialised to ``(0, bootstrap)``
(advantage_estimators.py:43-55), inputs promoted to at least float32
(:18-23), and

    delta = rho * (r + gamma * (1 - term) * V' - V) * (1 - trunc)      (:30-31)
    A     = delta + gamma * lam * c * (1 - term) * (1 - trunc) * A'     (:32-40)
    returns = A + V                                                    (:56)

Computed here in float64 unless ``dtype`` says otherwise.
"""
from __future__ import annotations

import numpy as np


def gae(reward, terminated, truncated, values, bootstrap, gamma, lam,
        rho=1.0, c=1.0, dtype=np.float64):
    reward = np.asarray(reward, dtype)
    values = np.asarray(values, dtype)
    bootstrap = np.asarray(bootstrap, dtype)
    term = np.asarray(terminated, dtype)
    trunc = np.asarray(truncated, dtype)
    rho = np.broadcast_to(np.asarray(rho, dtype), values.shape)
    c = np.broadcast_to(np.asarray(c, dtype), values.shape)
    gamma = dtype(gamma)
    lam = dtype(lam)
    adv = np.zeros_like(values)
    a = np.zeros_like(bootstrap)
    nv = bootstrap
    one = dtype(1.0)
    for t in range(values.shape[0] - 1, -1, -1):
        delta = rho[t] * (reward[t] + gamma * (one - term[t]) * nv - values[t])
        delta = delta * (one - trunc[t])
        a = delta + gamma * lam * c[t] * (one - term[t]) * (one - trunc[t]) * a
        adv[t] = a
        nv = values[t]
    return adv, adv + values
