"""Oracle of the linear-recurrence scan — TEST INFRASTRUCTURE ONLY.

Restates boonta/networks/kernels/scan.py's ``sequential`` (:117-131) forward
and the custom VJP of ``scan`` (:72-85) in float64 numpy:

    h_t = a_t h_{t-1} + b_t, h_{-1} = init
    db_t = g_t + a_{t+1} db_{t+1}, da_t = db_t h_{t-1}, dinit = db_0 a_0

``ssm_forward`` / ``ssm_vjp`` add the SSM block's episode reset in front of
the scan (boonta/networks/blocks/ssm.py:45-48).

Pinned by (tests/test_oracle_scan.py): the closed form
h_t = sum_s (prod_{s<r<=t} a_r) b_s + (prod_{r<=t} a_r) init on small inputs,
the special cases a = 1 (running sum) and a = 0 (h = b), linearity in
(b, init), and float64 central differences of sum(w * h) for both VJPs; the
reset by the reference torsos' invariant that a done step forgets everything
before it (tests/test_networks.py:51-66) and by done = False reducing to the
plain scan.  Only
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


def ssm_operands(a, b, done, reset=None):
    """The SSM block's reset (networks/blocks/ssm.py:45-48): where done,
    b' = b + a r and a' = 0 (r the restart carry, zeros by default)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    m = np.asarray(done, bool)[..., None].astype(np.float64)
    r = np.zeros((a.shape[0], a.shape[2])) if reset is None else np.asarray(reset, np.float64)
    return (1 - m) * a, b + m * a * r[:, None, :]


def ssm_forward(a, b, done, carry, reset=None):
    a2, b2 = ssm_operands(a, b, done, reset)
    return forward(a2, b2, carry)


def ssm_vjp(a, h, done, carry, g, reset=None):
    """(da, db, dcarry) of ssm_forward for the cotangent g of its output h."""
    a2, _ = ssm_operands(a, np.zeros_like(np.asarray(a, np.float64)), done, reset)
    da2, db2, dcarry = vjp(a2, h, carry, g)
    m = np.asarray(done, bool)[..., None].astype(np.float64)
    a = np.asarray(a, np.float64)
    r = np.zeros((a.shape[0], a.shape[2])) if reset is None else np.asarray(reset, np.float64)
    return (1 - m) * da2 + m * r[:, None, :] * db2, db2, dcarry
