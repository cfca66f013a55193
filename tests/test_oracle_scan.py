"""Pins the oracle's linear-recurrence scan (oracle/scan.py) by its closed
form, special cases, linearity and float64 finite differences of the VJP
(boonta/networks/kernels/scan.py:13-131)."""
import numpy as np

from oracle import scan


def closed_form(a, b, init):
    n, T, F = a.shape
    out = np.zeros((n, T, F))
    for t in range(T):
        acc = np.prod(a[:, : t + 1], axis=1) * init
        for s in range(t + 1):
            acc = acc + np.prod(a[:, s + 1: t + 1], axis=1) * b[:, s]
        out[:, t] = acc
    return out


def problem(seed, shape=(3, 7, 5)):
    rng = np.random.default_rng(seed)
    a = rng.uniform(0.05, 0.95, shape)
    b = rng.uniform(0, 1, shape)
    init = rng.standard_normal((shape[0], shape[2]))
    return a, b, init


def test_forward_is_the_closed_form():
    a, b, init = problem(0)
    np.testing.assert_allclose(scan.forward(a, b, init), closed_form(a, b, init), rtol=1e-12)


def test_special_cases():
    _, b, init = problem(1)
    np.testing.assert_allclose(scan.forward(np.ones_like(b), b, init), np.cumsum(b, axis=1) + init[:, None],
                               rtol=1e-12)
    np.testing.assert_array_equal(scan.forward(np.zeros_like(b), b, init), b)


def test_linear_in_b_and_init():
    a, b, init = problem(2)
    _, b2, init2 = problem(3)
    lhs = scan.forward(a, 2 * b - b2, 2 * init - init2)
    rhs = 2 * scan.forward(a, b, init) - scan.forward(a, b2, init2)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-10, atol=1e-12)


def test_vjp_matches_finite_differences():
    a, b, init = problem(4, (2, 6, 3))
    w = np.random.default_rng(5).standard_normal(a.shape)
    f = lambda a_, b_, i_: float(np.sum(w * scan.forward(a_, b_, i_)))
    da, db, dinit = scan.vjp(a, scan.forward(a, b, init), init, w)
    eps = 1e-6
    for arr, grad, which in ((a, da, 0), (b, db, 1), (init, dinit, 2)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            args = [a.copy(), b.copy(), init.copy()]
            args[which][idx] += eps
            up = f(*args)
            args[which][idx] -= 2 * eps
            num[idx] = (up - f(*args)) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)


def test_ssm_reset_forgets_the_past_and_reduces_to_the_scan():
    a, b, init = problem(6, (3, 9, 4))
    done = np.zeros((3, 9), bool)
    np.testing.assert_array_equal(scan.ssm_forward(a, b, done, init), scan.forward(a, b, init))
    done[:, 4] = True
    h = scan.ssm_forward(a, b, done, init)
    a2, b2, init2 = problem(7, (3, 9, 4))
    a2[:, 4:], b2[:, 4:] = a[:, 4:], b[:, 4:]
    h2 = scan.ssm_forward(a2, b2, done, init2)
    np.testing.assert_allclose(h[:, 4:], h2[:, 4:], rtol=1e-12)  # nothing before the reset matters
    reset = np.random.default_rng(8).standard_normal((3, 4))
    h3 = scan.ssm_forward(a, b, done, init, reset)
    np.testing.assert_allclose(h3[:, 4], a[:, 4] * reset + b[:, 4], rtol=1e-12)  # restarts from the reset carry


def test_ssm_vjp_matches_finite_differences():
    a, b, init = problem(9, (2, 6, 3))
    done = np.zeros((2, 6), bool)
    done[0, 0] = done[0, 3] = done[1, 5] = True
    reset = np.random.default_rng(10).standard_normal((2, 3))
    w = np.random.default_rng(11).standard_normal(a.shape)
    f = lambda a_, b_, i_: float(np.sum(w * scan.ssm_forward(a_, b_, done, i_, reset)))
    da, db, dinit = scan.ssm_vjp(a, scan.ssm_forward(a, b, done, init, reset), done, init, w, reset)
    eps = 1e-6
    for arr, grad, which in ((a, da, 0), (b, db, 1), (init, dinit, 2)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            args = [a.copy(), b.copy(), init.copy()]
            args[which][idx] += eps
            up = f(*args)
            args[which][idx] -= 2 * eps
            num[idx] = (up - f(*args)) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)
