"""Pins the oracle of RecurrentPuPO's prioritised env selection
(oracle/priority.py; boonta/algorithms/recurrent_pupo.py:226-236) by closed
forms and statistics rather than by re-typing its formulas."""
import numpy as np
import pytest

from boonta_amd.random import key as make_key
from oracle import priority, sample


def test_equal_priorities_follow_the_inverse_cdf_closed_form():
    # equal probabilities: c[n] = (n + 1) / N, r = 1 - u, first n with
    # c[n] >= r is N - 1 - floor(N u) (a forward draw r = u, or a 'right'
    # search, gives other indices)
    N, width = 10, 4096
    adv = np.ones((5, N))
    k = make_key(11)
    idx, w, prob, margin = priority.priority_choice(adv, k, width, 0.7, 0.4)
    u = sample.uniform(k, width, 0.0, 1.0).astype(np.float64)
    want = N - 1 - np.floor(N * u).astype(np.int64)
    ok = margin > 1e-9
    assert ok.mean() > 0.99
    np.testing.assert_array_equal(idx[ok], want[ok])
    np.testing.assert_allclose(prob, np.full(N, 1.0 / N), rtol=1e-6)   # the 1e-6 terms
    np.testing.assert_allclose(w, 1.0, rtol=1e-6)    # (N * 1/N) ** -beta


def test_a_single_env_with_all_the_priority_is_always_drawn():
    N = 64
    adv = np.zeros((8, N))
    adv[:, 17] = 3.0
    idx, w, prob, _ = priority.priority_choice(adv, make_key(5), 500, 1.0, 0.5)
    assert (idx == 17).all()
    assert prob[17] > 1 - 1e-6 * N
    np.testing.assert_allclose(w, (N * prob[17]) ** -0.5)


def test_priority_formula_on_a_hand_computed_case():
    # envs: |A| summed over time = 3, 1, 0 ; exponent 2 -> 9, 1, 0
    adv = np.array([[1.0, -1.0, 0.0], [-2.0, 0.0, 0.0]])
    np.testing.assert_allclose(priority.priorities(adv, 2.0), [9.0, 1.0, 0.0])
    np.testing.assert_allclose(priority.probabilities(adv, 2.0),
                               np.array([9 + 1e-6, 1 + 1e-6, 1e-6]) / (10 + 1e-6))


def test_draw_frequencies_match_the_probabilities():
    rng = np.random.default_rng(3)
    N, width = 12, 200_000
    adv = rng.standard_normal((6, N))
    idx, _, prob, _ = priority.priority_choice(adv, make_key(9), width, 0.6, 0.4)
    counts = np.bincount(idx, minlength=N)
    expected = width * prob
    chi2 = ((counts - expected) ** 2 / expected).sum()
    assert chi2 < 40.0   # 11 degrees of freedom: p < 1e-4 above 35


@pytest.mark.parametrize("beta", [0.0, 0.4, 1.0])
def test_importance_weights_closed_form(beta):
    rng = np.random.default_rng(4)
    adv = rng.standard_normal((4, 30))
    idx, w, prob, _ = priority.priority_choice(adv, make_key(1), 100, 0.6, beta)
    np.testing.assert_allclose(w, (30 * prob[idx]) ** -beta)
    if beta == 0.0:
        np.testing.assert_allclose(w, 1.0)


@pytest.mark.parametrize("T,N,width,exponent,most", [
    (64, 1024, 256, 0.6, 0), (7, 1000, 1000, 1.0, 0), (2, 16384, 4096, 0.5, 25), (16, 3000, 20000, 0.8, 24)])
def test_float64_running_sum_against_jax_float32_typing(T, N, width, exponent, most):
    """The product's draw searches a float64 running sum of the float32
    probabilities; jax 0.10.2 types the cumsum and r in float32.  On the GPU
    test cases the two agree on every draw at the recurrent workload's shape
    and otherwise differ on at most ``most`` draws (0.6 %), each by one env."""
    rng = np.random.default_rng(T * 7919 + N)
    adv = (rng.standard_normal((T, N)) * rng.uniform(0.1, 3.0, N)).astype(np.float32)
    k = make_key(1000 + N)
    prob = priority.probabilities(adv, exponent).astype(np.float32)
    i64, _ = priority.choice(k, prob.astype(np.float64), width)
    i32 = priority.choice_f32(k, prob, width)
    assert (i64 != i32).sum() <= most
    assert np.abs(i64 - i32).max() <= 1


def test_float32_choice_follows_the_inverse_cdf_closed_form():
    # equal probabilities over 10 envs: N - 1 - floor(N u) wherever N u is not
    # within float32 rounding of an integer
    N, width = 10, 4096
    k = make_key(12)
    u = sample.uniform(k, width, 0.0, 1.0).astype(np.float64)
    eq = priority.choice_f32(k, np.full(N, 1.0 / N, np.float32), width)
    want = N - 1 - np.floor(N * u).astype(np.int64)
    far = np.abs(N * u - np.round(N * u)) > 1e-5
    assert far.mean() > 0.99
    np.testing.assert_array_equal(eq[far], want[far])
