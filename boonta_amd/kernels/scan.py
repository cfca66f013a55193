"""Linear-recurrence scan h_t = a_t h_{t-1} + b_t on MI355X, with its
vector-Jacobian product, mirroring boonta/networks/kernels/scan.py:

- ``scan(a, b, init)`` (:72-88): a [batch, steps, features], init [batch,
  features]; differentiable (a ``torch.autograd.Function`` whose forward and
  backward are ``ppo_linear_scan_fwd`` / ``ppo_linear_scan_bwd``), returning
  the operands' dtype (float32 or bfloat16 storage, float32 accumulation);
- ``hip(a, b, init)`` (the reference's ``pallas``, :91-101): also takes
  extra axes between steps and features, [batch, steps, *extra, features],
  folded into the batch;
- ``get_scan_implementation(name)``: the lookup the SSM block uses
  (networks/blocks/ssm.py:49).

There is no CPU path: the kernels run on the device the tensors live on.
"""
from __future__ import annotations

import torch

from .. import _lib

_DTYPES = {torch.float32: 0, torch.bfloat16: 1}


def _check(a, b, init):
    if a.dtype not in _DTYPES:
        raise TypeError(f"the scan stores float32 or bfloat16, not {a.dtype}")
    if b.dtype != a.dtype or init.dtype != a.dtype:
        raise TypeError("a, b and init must share one dtype")
    if a.dim() != 3 or b.shape != a.shape or init.shape != (a.shape[0], a.shape[2]):
        raise ValueError(f"need a, b [batch, steps, features] and init [batch, features]; got "
                         f"{tuple(a.shape)}, {tuple(b.shape)}, {tuple(init.shape)}")
    if not (a.is_cuda and b.is_cuda and init.is_cuda):
        raise TypeError("the scan runs on device tensors")


def _stream():
    return torch.cuda.current_stream().cuda_stream


class _LinearScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, init):
        a, b, init = a.contiguous(), b.contiguous(), init.contiguous()
        out = torch.empty_like(a)
        n, t, f = a.shape
        _lib.call("ppo_linear_scan_fwd", _stream(), _DTYPES[a.dtype], a.data_ptr(), b.data_ptr(), init.data_ptr(),
                  out.data_ptr(), n, t, f)
        ctx.save_for_backward(a, out, init)
        return out

    @staticmethod
    def backward(ctx, g):
        a, h, init = ctx.saved_tensors
        g = g.to(a.dtype).contiguous()
        da, db, dinit = torch.empty_like(a), torch.empty_like(a), torch.empty_like(init)
        n, t, f = a.shape
        _lib.call("ppo_linear_scan_bwd", _stream(), _DTYPES[a.dtype], a.data_ptr(), h.data_ptr(), init.data_ptr(),
                  g.data_ptr(), da.data_ptr(), db.data_ptr(), dinit.data_ptr(), n, t, f)
        return da, db, dinit


def scan(a: torch.Tensor, b: torch.Tensor, init: torch.Tensor) -> torch.Tensor:
    _check(a, b, init)
    return _LinearScan.apply(a, b, init)


def hip(a: torch.Tensor, b: torch.Tensor, init: torch.Tensor) -> torch.Tensor:
    """[batch, steps, *extra, features] operands, init [batch, *extra, features]."""
    if a.dim() == 3:
        return scan(a, b, init)
    batch, steps, *extra, features = a.shape

    def fold(x):
        return torch.movedim(x, 1, -2).reshape(-1, steps, features)

    out = scan(fold(a), fold(b), init.reshape(-1, features))
    return torch.movedim(out.reshape(batch, *extra, steps, features), -2, 1)


_IMPLEMENTATIONS = {"hip": hip}


def get_scan_implementation(name: str = "hip"):
    if name not in _IMPLEMENTATIONS:
        raise NotImplementedError(f"scan implementation {name!r} is not compiled (available: hip)")
    return _IMPLEMENTATIONS[name]
