"""RecurrentPuPO's prioritised env selection on the GPU: the drop-in for the
minibatch selection of boonta/algorithms/recurrent_pupo.py:226-236.

``prioritized_choice(advantages, key, width, priority_exponent, beta)``
returns what ``minibatch_fn`` computes from the V-trace advantages before it
gathers the minibatch: the env indices ``jax.random.choice(key, num_envs,
(width,), replace=True, p=probabilities)``, the importance weights
``(num_envs * probabilities[indices]) ** -beta`` and the probabilities
themselves, in one launch of ``ppo_priority_choice_f32``.  The V-trace
advantages come from ``generalized_advantage_estimator`` with per-element
``rho = min(ratio, advantage_clip)`` and ``c = min(ratio, trace_clip)``
(recurrent_pupo.py:210-220), which ``ppo_gae_f32`` takes as arrays.
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _lib
from ..random import key_data


def prioritized_choice(advantages: torch.Tensor, key, width: int, priority_exponent: float, beta: float):
    """advantages: float32 device tensor [T, N] (time-major, unit column
    stride); key: key data (host) or a device tensor of two 32-bit words.
    Returns (indices int32 [width], weights float32 [width], probabilities
    float32 [N]) on the current stream."""
    if not (isinstance(advantages, torch.Tensor) and advantages.is_cuda and advantages.dtype == torch.float32):
        raise TypeError("advantages must be a float32 device tensor")
    if advantages.dim() != 2 or advantages.stride(1) != 1:
        raise ValueError("advantages must be [T, N] with unit column stride")
    T, N = advantages.shape
    dev = advantages.device
    if isinstance(key, torch.Tensor) and key.is_cuda:
        if key.numel() != 2 or key.element_size() != 4:
            raise ValueError("a device key must hold two 32-bit words")
        kd = key.reshape(2).view(torch.int32)
    else:
        kd = torch.from_numpy(key_data(key).view(np.int32).copy()).to(dev)
    indices = torch.empty(width, dtype=torch.int32, device=dev)
    weights = torch.empty(width, dtype=torch.float32, device=dev)
    probabilities = torch.empty(N, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    _lib.call("ppo_priority_choice_f32", st, advantages.data_ptr(), advantages.stride(0), T, N,
              float(priority_exponent), float(beta), kd.data_ptr(), width, indices.data_ptr(), weights.data_ptr(),
              probabilities.data_ptr())
    return indices, weights, probabilities
