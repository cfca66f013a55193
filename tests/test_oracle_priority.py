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
