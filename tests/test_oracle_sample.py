"""Pins the oracle's rollout sampling (oracle/sample.py) by what the
mathematics fixes: the uniform map's endpoints on hand-computed words, the
Gumbel-max frequencies against softmax probabilities, the normal draws'
moments and distribution, log-probabilities against independent library
routines, and the greedy case (boonta/networks/distributions.py:8-57)."""
import numpy as np
import pytest
from scipy import special, stats

from oracle import prng, sample

F32 = np.float32


def test_uniform_endpoints_on_hand_computed_words():
    words = np.array([0, 0x200, 0x80000000, 0xFFFFFFFF], np.uint32)
    u = sample.words_to_uniform(words, sample.TINY32, 1.0)
    assert u.dtype == np.float32
    np.testing.assert_array_equal(u, np.array([sample.TINY32, 2.0 ** -23, 0.5, 1 - 2.0 ** -23], F32))
    v = sample.words_to_uniform(words, sample.NEXT_ABOVE_MINUS_ONE, 1.0)
    # (maxval - minval) rounds to 2 in float32, so u = 2 f - 1 + 2^-24
    np.testing.assert_array_equal(v, np.array([-1 + 2.0 ** -24, -1 + 2.0 ** -24 + 2.0 ** -22, 2.0 ** -24,
                                               1 - 3 * 2.0 ** -24], F32))
    assert float(sample.NEXT_ABOVE_MINUS_ONE) == -1 + 2.0 ** -24


def test_uniform_reads_the_keys_word_stream():
    k = prng.key(7)
    u = sample.uniform(k, 1000, 0.0, 1.0)
    bits = prng.random_bits32(k, 1000)
    np.testing.assert_array_equal(u, (bits >> 9).astype(np.float64) * 2.0 ** -23)
    assert u.min() >= 0 and u.max() < 1


@pytest.mark.parametrize("temperature", [1.0, 2.0, 0.5])
def test_gumbel_max_frequencies_follow_softmax(temperature):
    p = np.array([0.1, 0.2, 0.3, 0.4])
    rows = 40000
    pref = np.broadcast_to(np.log(p), (rows, 4))
    a, lp, _ = sample.categorical_sample(pref, prng.key(123), temperature)
    q = p ** (1 / temperature)
    q /= q.sum()
    counts = np.bincount(a, minlength=4)
    assert stats.chisquare(counts, q * rows).pvalue > 1e-3
    np.testing.assert_allclose(lp, np.log(q)[a], rtol=1e-12)


def test_categorical_log_prob_and_tie_margin():
    rng = np.random.default_rng(0)
    pref = rng.standard_normal((500, 7)) * 3
    a, lp, margin = sample.categorical_sample(pref, prng.key(5), 1.0)
    ls = pref - pref.max(-1, keepdims=True)
    ls = ls - np.log(np.exp(ls).sum(-1, keepdims=True))
    np.testing.assert_allclose(lp, ls[np.arange(500), a], rtol=1e-12)
    z = ls + sample.gumbel(prng.key(5), 500 * 7).reshape(500, 7)
    np.testing.assert_array_equal(a, z.argmax(-1))
    assert np.all(margin >= 0)


def test_greedy_at_zero_temperature():
    rng = np.random.default_rng(1)
    pref = rng.standard_normal((300, 5))
    a, lp, _ = sample.categorical_sample(pref, prng.key(9), 0.0)
    np.testing.assert_array_equal(a, pref.argmax(-1))
    np.testing.assert_array_equal(lp, 0.0)


def test_normal_draws_are_standard_normal():
    n = 200000
    eps = sample.normal(prng.key(11), n)
    assert abs(eps.mean()) < 5 / np.sqrt(n)
    assert abs(eps.var() - 1) < 0.01
    assert stats.kstest(eps, "norm").pvalue > 1e-3
    u = sample.uniform(prng.key(11), n, sample.NEXT_ABOVE_MINUS_ONE, 1.0).astype(np.float64)
    np.testing.assert_allclose(eps, stats.norm.ppf((u + 1) / 2), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("temperature", [1.0, 0.3])
def test_gaussian_log_prob_is_the_normal_density(temperature):
    rng = np.random.default_rng(2)
    mean = rng.standard_normal((400, 8))
    raw = rng.standard_normal((400, 8))
    a, lp, eps = sample.gaussian_sample(mean, raw, prng.key(3), temperature)
    sig = temperature * (np.log1p(np.exp(raw)) + 1e-3)
    np.testing.assert_allclose(a, sig * eps + mean, rtol=1e-12)
    np.testing.assert_allclose(lp, stats.norm.logpdf(a, mean, sig).sum(-1), rtol=1e-9, atol=1e-9)
    # state-independent scale: one vector broadcast over rows
    s = rng.standard_normal(8)
    a2, lp2, eps2 = sample.gaussian_sample(mean, s, prng.key(3), temperature)
    np.testing.assert_array_equal(eps2, eps)
    sig2 = temperature * (np.log1p(np.exp(s)) + 1e-3)
    np.testing.assert_allclose(lp2, stats.norm.logpdf(a2, mean, sig2).sum(-1), rtol=1e-9, atol=1e-9)


def test_erfinv_identity_used_by_the_normal():
    x = np.linspace(-0.999999, 0.999999, 10001)
    np.testing.assert_allclose(special.erf(special.erfinv(x)), x, atol=1e-12)
