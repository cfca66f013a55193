"""RecurrentPuPO's prioritised env selection on the GPU: the drop-in for the
minibatch selection of boonta/algorithms/recurrent_pupo.py:226-236.

``prioritized_choice(advantages, key, width, priority_exponent, beta)``
returns what ``minibatch_fn`` computes from the V-trace advantages before it
gathers the minibatch: the env indices ``jax.random.choice(key, num_envs,
(width,), replace=True, p=probabilities)``, the importance weights
``(num_envs * probabilities[indices]) ** -beta`` and the probabilities
themselves, in one launch of ``ppo_priority_choice_f32``.

``vtrace(...)`` is the ``vtrace`` closure of recurrent_pupo.py:210-220: the
advantage estimator with ``rho = min(ratio, advantage_clip)`` and
``c = min(ratio, trace_clip)`` on the env-major ratio, in one launch of
``ppo_vtrace_f32`` (the GAE scan forming the clipped weights as it reads them).
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


def _u8(x):
    return x.to(torch.uint8).contiguous()


def vtrace(reward: torch.Tensor, terminated: torch.Tensor, truncated: torch.Tensor, values: torch.Tensor,
           bootstrap: torch.Tensor, ratio: torch.Tensor, gamma: float, gae_lambda: float, advantage_clip: float,
           trace_clip: float, chunks: int = 0):
    """reward / values float32 [T, N], terminated / truncated bool [T, N],
    bootstrap [N], ratio float32 [N, T] (env-major, unit column stride), all
    on the device.  Returns (advantages, returns) float32 [T, N]."""
    T, N = reward.shape
    if ratio.dim() != 2 or ratio.shape[0] != N or ratio.shape[1] != T or ratio.stride(1) != 1:
        raise ValueError("ratio must be [N, T] with unit column stride")
    f32 = [x.to(torch.float32).contiguous() for x in (reward, values, bootstrap)]
    if ratio.dtype != torch.float32:
        raise TypeError("ratio must be float32")
    te, tr = _u8(terminated), _u8(truncated)
    adv = torch.empty(T, N, dtype=torch.float32, device=reward.device)
    ret = torch.empty_like(adv)
    st = torch.cuda.current_stream(reward.device).cuda_stream
    _lib.call("ppo_vtrace_f32", st, f32[0].data_ptr(), te.data_ptr(), tr.data_ptr(), f32[1].data_ptr(),
              f32[2].data_ptr(), ratio.data_ptr(), ratio.stride(0), float(advantage_clip), float(trace_clip),
              adv.data_ptr(), ret.data_ptr(), T, N, float(gamma), float(gae_lambda), chunks)
    return adv, ret
