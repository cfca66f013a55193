"""GAE on the GPU: the drop-in for boonta/algorithms/advantage_estimators.py:8-56.

``generalized_advantage_estimator(transitions, values, bootstrap, gamma,
gae_lambda, rho=1.0, c=1.0) -> (advantages, returns)`` keeps the reference's
signature and runs the HIP reverse scan ``ppo_gae_f32`` on the current torch
stream.  Inputs are promoted to float32 as the reference promotes them to at
least float32 (advantage_estimators.py:18-23); float64 inputs are not
compiled and raise.
"""
from __future__ import annotations

import torch

from .. import _lib


def _f32(x, like):
    t = x if isinstance(x, torch.Tensor) else torch.as_tensor(x, device=like.device)
    if t.dtype == torch.float64:
        raise NotImplementedError("float64 GAE is not compiled")
    return t.to(device=like.device, dtype=torch.float32).contiguous()


def generalized_advantage_estimator(transitions, values, bootstrap, gamma: float, gae_lambda: float,
                                    rho=1.0, c=1.0, chunks: int = 0):
    reward = transitions.second.reward
    T, N = reward.shape[:2]
    reward = _f32(reward, reward)
    values = _f32(values, reward)
    bootstrap = _f32(bootstrap, reward)
    term = transitions.second.terminated.to(device=reward.device, dtype=torch.bool).contiguous()
    trunc = transitions.second.truncated.to(device=reward.device, dtype=torch.bool).contiguous()
    rho_t = None if (not isinstance(rho, torch.Tensor) and rho == 1.0) else \
        torch.broadcast_to(_f32(rho, reward), (T, N)).contiguous()
    c_t = None if (not isinstance(c, torch.Tensor) and c == 1.0) else \
        torch.broadcast_to(_f32(c, reward), (T, N)).contiguous()
    adv = torch.empty(T, N, dtype=torch.float32, device=reward.device)
    ret = torch.empty_like(adv)
    st = torch.cuda.current_stream(reward.device).cuda_stream
    _lib.call("ppo_gae_f32", st, reward.data_ptr(), term.data_ptr(), trunc.data_ptr(), values.data_ptr(),
              bootstrap.data_ptr(), None if rho_t is None else rho_t.data_ptr(),
              None if c_t is None else c_t.data_ptr(), adv.data_ptr(), ret.data_ptr(), T, N, float(gamma),
              float(gae_lambda), int(chunks))
    return adv, ret
