"""Pins the oracle GAE (oracle/gae.py) with closed forms and the reference's
own test construction (tests/test_algorithms.py:145-214 of the reference:
rng(0), shape (6, 3), gamma 0.9, lambda 0.8, terminated p=0.2, truncated
p=0.2 and not terminated, V-trace rho, c ~ U(0.5, 1.5))."""
import numpy as np
import pytest

from oracle.gae import gae


def reference_case(weighted):
    g = np.random.default_rng(0)
    shape = (6, 3)
    reward, values = g.normal(size=shape), g.normal(size=shape)
    bootstrap = g.normal(size=shape[1:])
    terminated = g.random(shape) < 0.2
    truncated = (g.random(shape) < 0.2) & ~terminated
    rho, c = (g.uniform(0.5, 1.5, shape) if weighted else np.ones(shape) for _ in range(2))
    return reward, values, bootstrap, terminated, truncated, rho, c


def test_no_dones_is_the_discounted_sum_of_deltas():
    g = np.random.default_rng(1)
    T, N = 9, 4
    r, v, b = g.normal(size=(T, N)), g.normal(size=(T, N)), g.normal(size=N)
    z = np.zeros((T, N), bool)
    adv, ret = gae(r, z, z, v, b, 0.97, 0.9)
    vnext = np.concatenate([v[1:], b[None]], 0)
    delta = r + 0.97 * vnext - v
    expect = np.array([sum((0.97 * 0.9) ** (k - t) * delta[k] for k in range(t, T)) for t in range(T)])
    np.testing.assert_allclose(adv, expect, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ret, expect + v, rtol=1e-12)


def test_lambda_zero_is_the_one_step_td_error():
    r, v, b, te, tr, _, _ = reference_case(False)
    adv, _ = gae(r, te, tr, v, b, 0.9, 0.0)
    vnext = np.concatenate([v[1:], b[None]], 0)
    np.testing.assert_allclose(adv, (r + 0.9 * (1 - te) * vnext - v) * (1 - tr), atol=1e-12)


def test_truncation_zeroes_the_advantage_and_returns_the_value():
    r, v, b, te, tr, _, _ = reference_case(False)
    adv, ret = gae(r, te, tr, v, b, 0.9, 0.8)
    assert tr.any()
    np.testing.assert_array_equal(adv[tr], 0.0)
    np.testing.assert_array_equal(ret[tr], v[tr])


def test_termination_cuts_the_bootstrap_and_the_carry():
    r, v, b, te, tr, _, _ = reference_case(False)
    adv, _ = gae(r, te, tr, v, b, 0.9, 0.8)
    assert te.any()
    np.testing.assert_allclose(adv[te], (r - v)[te], atol=1e-12)


def test_an_episode_boundary_hides_the_future():
    r, v, b, te, tr, _, _ = reference_case(False)
    te = np.zeros_like(te)
    tr = np.zeros_like(tr)
    te[2] = True
    a1, _ = gae(r, te, tr, v, b, 0.9, 0.8)
    r2, v2 = r.copy(), v.copy()
    r2[3:] += 50.0
    v2[3:] -= 7.0
    a2, _ = gae(r2, te, tr, v2, b + 3.0, 0.9, 0.8)
    np.testing.assert_allclose(a1[:3], a2[:3], atol=1e-12)


@pytest.mark.parametrize("weighted", [False, True], ids=["gae", "vtrace"])
def test_vtrace_weights_scale_delta_and_carry(weighted):
    r, v, b, te, tr, rho, c = reference_case(weighted)
    adv, _ = gae(r, te, tr, v, b, 0.9, 0.8, rho=rho, c=c)
    # last step: no carry, delta scaled by rho
    last = rho[-1] * (r[-1] + 0.9 * (1 - te[-1]) * b - v[-1]) * (1 - tr[-1])
    np.testing.assert_allclose(adv[-1], last, atol=1e-12)
    # one step earlier: carry weighted by c
    d = rho[-2] * (r[-2] + 0.9 * (1 - te[-2]) * v[-1] - v[-2]) * (1 - tr[-2])
    np.testing.assert_allclose(adv[-2], d + 0.9 * 0.8 * c[-2] * (1 - te[-2]) * (1 - tr[-2]) * last,
                               atol=1e-12)


def test_bf16_like_inputs_promote_to_float32():
    adv, ret = gae(np.ones((4, 2)), np.zeros((4, 2), bool), np.zeros((4, 2), bool), np.ones((4, 2)),
                   np.ones(2), 0.99, 0.95, dtype=np.float32)
    assert adv.dtype == ret.dtype == np.float32
