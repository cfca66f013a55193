"""Oracle PRNG: ctypes view of ``oracle/threefry.c`` (test infrastructure only).

Restates jax 0.10.2's ``jax.random.key``/``split``/``permutation`` as called by
boonta/algorithms/ppo.py:199-201,230-231 and recurrent_ppo.py:269-279.  Only
``tests/``, ``bench.py``'s CPU baseline and ``__graft_entry__.smoke`` use it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = ctypes.CDLL(_LIB)
        u32p = ctypes.POINTER(ctypes.c_uint32)
        i32p = ctypes.POINTER(ctypes.c_int32)
        L.oracle_threefry2x32.argtypes = [ctypes.c_uint32] * 4 + [u32p]
        L.oracle_split.argtypes = [u32p, ctypes.c_int64, u32p]
        L.oracle_random_bits32.argtypes = [u32p, ctypes.c_int64, u32p]
        L.oracle_shuffle_rounds.argtypes = [ctypes.c_int64]
        L.oracle_shuffle_rounds.restype = ctypes.c_int
        L.oracle_stable_sort_by_key.argtypes = [u32p, i32p, ctypes.c_int64]
        L.oracle_permutation.argtypes = [u32p, ctypes.c_int64, i32p]
        L.oracle_epoch_permutations.argtypes = [u32p, ctypes.c_int, ctypes.c_int64, i32p]
        _lib = L
    return _lib


def _u32(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def _i32(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def key(seed: int) -> np.ndarray:
    """``jax.random.key(seed)`` key data: (seed >> 32, seed & 0xffffffff)."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    return np.array([seed >> 32, seed & 0xFFFFFFFF], dtype=np.uint32)


def threefry2x32(k0: int, k1: int, x0: int, x1: int) -> tuple[int, int]:
    out = np.zeros(2, np.uint32)
    lib().oracle_threefry2x32(k0, k1, x0, x1, _u32(out)[1])
    return int(out[0]), int(out[1])


def split(k: np.ndarray, num: int = 2) -> np.ndarray:
    k, kp = _u32(k)
    out = np.zeros((num, 2), np.uint32)
    lib().oracle_split(kp, num, _u32(out)[1])
    return out


def random_bits32(k: np.ndarray, n: int) -> np.ndarray:
    k, kp = _u32(k)
    out = np.zeros(n, np.uint32)
    lib().oracle_random_bits32(kp, n, _u32(out)[1])
    return out


def shuffle_rounds(n: int) -> int:
    return int(lib().oracle_shuffle_rounds(n))


def stable_sort_by_key(keys: np.ndarray, vals: np.ndarray) -> np.ndarray:
    keys, kp = _u32(keys)
    vals = np.ascontiguousarray(vals, dtype=np.int32).copy()
    lib().oracle_stable_sort_by_key(kp, _i32(vals), len(vals))
    return vals


def permutation(k: np.ndarray, n: int) -> np.ndarray:
    k, kp = _u32(k)
    out = np.zeros(n, np.int32)
    lib().oracle_permutation(kp, n, _i32(out))
    return out


def epoch_permutations(k: np.ndarray, epochs: int, n: int) -> np.ndarray:
    """Rows of ``permutation(split(k, epochs)[e], n)``: ppo.py:200,230."""
    k, kp = _u32(k)
    out = np.zeros((epochs, n), np.int32)
    lib().oracle_epoch_permutations(kp, epochs, n, _i32(out))
    return out
