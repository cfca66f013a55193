"""PRNG keys of the learner: jax.random.key(seed) key data (threefry2x32).

A key is two uint32 words, (seed >> 32, seed & 0xffffffff).  Splitting and the
epoch permutations run on the GPU (``ppo_threefry_split``,
``ppo_epoch_permutations``); this module only builds and normalises key data.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib


def key(seed: int) -> np.ndarray:
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    return np.array([seed >> 32, seed & 0xFFFFFFFF], dtype=np.uint32)


PRNGKey = key


def key_data(k) -> np.ndarray:
    """uint32[2] key data of an int seed, a key array, or a tensor of key data."""
    if isinstance(k, (int, np.integer)):
        return key(int(k))
    if isinstance(k, torch.Tensor):
        k = k.detach().cpu().numpy()
    a = np.asarray(k)
    if a.shape != (2,):
        raise ValueError(f"key data must have shape (2,), got {a.shape}")
    return a.astype(np.int64).astype(np.uint32) if a.dtype != np.uint32 else a.copy()


def split(k, num: int = 2, device="cuda") -> np.ndarray:
    """jax.random.split(key, num) computed by the HIP kernel; returns uint32 [num, 2]."""
    kd = torch.from_numpy(key_data(k).view(np.int32).copy()).to(device)
    out = torch.empty(num, 2, dtype=torch.int32, device=device)
    _lib.call("ppo_threefry_split", torch.cuda.current_stream().cuda_stream, kd.data_ptr(), out.data_ptr(), num)
    return out.cpu().numpy().view(np.uint32)


def permutation(k, n: int, device="cuda") -> torch.Tensor:
    """jax.random.permutation(key, n) computed on the GPU (int32 device tensor)."""
    kd = torch.from_numpy(key_data(k).view(np.int32).copy()).to(device)
    out = torch.empty(n, dtype=torch.int32, device=device)
    ws = torch.empty(_lib.load().ppo_permutation_workspace(n), dtype=torch.uint8, device=device)
    _lib.call("ppo_permutation", torch.cuda.current_stream().cuda_stream, kd.data_ptr(), out.data_ptr(), n,
              ws.data_ptr(), ws.numel())
    return out
