"""Pins the oracle's PRNG restatement (oracle/threefry.c).

- Threefry-2x32-20 against the Random123 known-answer vectors (the same three
  vectors jax's own threefry test uses).
- split(key(0)) against the value jax's documentation prints for
  ``jax.random.split(jax.random.key(0))`` under the partitionable threefry.
- the stable sort against numpy's stable argsort, the round count against its
  closed form, and permutation invariants.
"""
import math

import numpy as np
import pytest

from oracle import prng


@pytest.mark.parametrize("key, ctr, expected", [
    ((0x00000000, 0x00000000), (0x00000000, 0x00000000), (0x6B200159, 0x99BA4EFE)),
    ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF), (0x1CB996FC, 0xBB002BE7)),
    ((0x13198A2E, 0x03707344), (0x243F6A88, 0x85A308D3), (0xC4923A9C, 0x483DF7A0)),
])
def test_threefry_matches_random123_known_answers(oracle_lib, key, ctr, expected):
    assert prng.threefry2x32(*key, *ctr) == expected


def test_split_of_key_zero_matches_the_documented_value(oracle_lib):
    np.testing.assert_array_equal(prng.split(prng.key(0), 2),
                                  np.array([[1797259609, 2579123966], [928981903, 3453687069]], np.uint32))


def test_key_holds_the_seed_words(oracle_lib):
    np.testing.assert_array_equal(prng.key(42), [0, 42])
    np.testing.assert_array_equal(prng.key((7 << 32) | 5), [7, 5])


def test_split_counter_layout(oracle_lib):
    k = prng.key(1234)
    out = prng.split(k, 5)
    for i in range(5):
        assert tuple(out[i]) == prng.threefry2x32(int(k[0]), int(k[1]), 0, i)


def test_random_bits_xor_the_two_words(oracle_lib):
    k = prng.key(7)
    bits = prng.random_bits32(k, 9)
    for i in range(9):
        a, b = prng.threefry2x32(int(k[0]), int(k[1]), 0, i)
        assert bits[i] == (a ^ b)


@pytest.mark.parametrize("n", [0, 1, 2, 100, 1000, 1023, 1024, 1025, 2048, 65536, 262144])
def test_round_count_closed_form(oracle_lib, n):
    expected = int(np.ceil(3 * np.log(max(1, n)) / np.log(np.iinfo(np.uint32).max)))
    assert prng.shuffle_rounds(n) == expected


def test_round_count_boundary(oracle_lib):
    # one round up to n = floor((2^32-1)^(1/3)) = 1625, two rounds after
    assert prng.shuffle_rounds(1625) == 1
    assert prng.shuffle_rounds(1626) == 2


def test_stable_sort_matches_numpy_stable_argsort(oracle_lib):
    rng = np.random.default_rng(0)
    keys = rng.integers(0, 16, 5000).astype(np.uint32)  # many ties
    vals = np.arange(5000, dtype=np.int32)[::-1].copy()
    out = prng.stable_sort_by_key(keys, vals)
    np.testing.assert_array_equal(out, vals[np.argsort(keys, kind="stable")])


@pytest.mark.parametrize("n", [1, 7, 512, 3000, 65536])
def test_permutation_is_a_permutation(oracle_lib, n):
    p = prng.permutation(prng.key(3), n)
    np.testing.assert_array_equal(np.sort(p), np.arange(n))


def test_permutation_composes_split_bits_and_sort(oracle_lib):
    n = 3000  # two rounds
    k = prng.key(11)
    x = np.arange(n, dtype=np.int32)
    for _ in range(prng.shuffle_rounds(n)):
        k, sub = prng.split(k, 2)
        x = x[np.argsort(prng.random_bits32(sub, n), kind="stable")]
    np.testing.assert_array_equal(prng.permutation(prng.key(11), n), x)


def test_epoch_permutations_use_split_keys(oracle_lib):
    k = prng.key(5)
    out = prng.epoch_permutations(k, 3, 777)
    keys = prng.split(k, 3)
    for e in range(3):
        np.testing.assert_array_equal(out[e], prng.permutation(keys[e], 777))
    assert len({tuple(r[:20]) for r in out}) == 3
