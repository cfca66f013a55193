"""Oracle of the linear-recurrence scan — TEST INFRASTRUCTURE ONLY.

Restates boonta/networks/kernels/scan.py's ``sequential`` (:117-131) forward
and the custom VJP of ``scan`` (:72-85) in float64 numpy:

    h_t = a_t h_{t-1} + b_t, h_{-1} = init
    db_t = g_t + a_{t+1} db_{t+1}, da_t = db_t h_{t-1}, dinit = db_0 a_0

Pinned by (tests/test_oracle_scan.py): the closed form
h_t = sum_s (prod_{s<r<=t} a_r) b_s + (prod_{r<=t} a_r) init on small inputs,
the special cases a = 1 (running sum) and a = 0 (h = b), linearity in
(b, init), and float64 central differences of sum(w * h) for the VJP.  Only
``tests/`` and ``bench.py``'s CPU baseline use it.
"""
from __future__ import annotations

import numpy as np


def forward(a, b, init):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    h = np.asarray(init, np.float64).copy()
    out = np.empty_like(a)
    for t in range(a.shape[1]):
        h = a[:, t] * h + b[:, t]
        out[:, t] = h
    return out


def vjp(a, h, init, g):
    """(da, db, dinit) for the cotangent g of the forward's output h."""
    a = np.asarray(a, np.float64)
    h = np.asarray(h, np.float64)
    g = np.asarray(g, np.float64)
    steps = a.shape[1]
    db = np.empty_like(g)
    d = np.zeros_like(g[:, 0])
    for t in range(steps - 1, -1, -1):
        nxt = a[:, t + 1] if t + 1 < steps else 0.0
        d = g[:, t] + nxt * d
        db[:, t] = d
    shifted = np.concatenate([np.asarray(init, np.float64)[:, None], h[:, :-1]], axis=1)
    return db * shifted, db, db[:, 0] * a[:, 0]
