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
  (networks/blocks/ssm.py:49);
- ``ssm(a, b, done, carry, reset)`` / ``ssm_scan``: the SSM block's episode
  reset folded into the same launches (ssm.py:40-55).

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


class _SSMScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, done, carry, reset):
        a, b, carry = a.contiguous(), b.contiguous(), carry.contiguous()
        done = done.contiguous()
        reset = None if reset is None else reset.contiguous()
        out = torch.empty_like(a)
        n, t, f = a.shape
        _lib.call("ppo_ssm_scan_fwd", _stream(), _DTYPES[a.dtype], a.data_ptr(), b.data_ptr(), done.data_ptr(),
                  None if reset is None else reset.data_ptr(), carry.data_ptr(), out.data_ptr(), n, t, f)
        ctx.save_for_backward(a, out, done, carry, reset)
        return out

    @staticmethod
    def backward(ctx, g):
        a, h, done, carry, reset = ctx.saved_tensors
        g = g.to(a.dtype).contiguous()
        da, db, dcarry = torch.empty_like(a), torch.empty_like(a), torch.empty_like(carry)
        n, t, f = a.shape
        _lib.call("ppo_ssm_scan_bwd", _stream(), _DTYPES[a.dtype], a.data_ptr(), h.data_ptr(), done.data_ptr(),
                  None if reset is None else reset.data_ptr(), carry.data_ptr(), g.data_ptr(), da.data_ptr(),
                  db.data_ptr(), dcarry.data_ptr(), n, t, f)
        return da, db, None, dcarry, None


def ssm_scan(a: torch.Tensor, b: torch.Tensor, done: torch.Tensor, carry: torch.Tensor,
             reset: torch.Tensor | None = None) -> torch.Tensor:
    """The carries of boonta's SSM block (networks/blocks/ssm.py:40-51): where
    ``done`` [batch, steps] (bool), the step restarts from ``reset`` (the cell's
    initial carry; None: zeros) — b' = b + a reset, a' = 0 — then the scan from
    ``carry``; one launch forward, one backward (``reset`` gets no gradient,
    like the cell's constant initial carry)."""
    _check(a, b, carry)
    if done.dtype != torch.bool or tuple(done.shape) != tuple(a.shape[:2]) or not done.is_cuda:
        raise ValueError("done must be a bool [batch, steps] device tensor")
    if reset is not None and (reset.dtype != a.dtype or reset.shape != carry.shape):
        raise ValueError("reset must match carry's shape and the operands' dtype")
    return _SSMScan.apply(a, b, done, carry, reset)


def ssm(a: torch.Tensor, b: torch.Tensor, done: torch.Tensor, carry: torch.Tensor,
        reset: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(final carry [batch, features], carries [batch, steps, features]), as
    SSM.__call__ returns them before the cell's output map (ssm.py:51-55)."""
    carries = ssm_scan(a, b, done, carry, reset)
    return carries[:, -1], carries


_IMPLEMENTATIONS = {"hip": hip}


def get_scan_implementation(name: str = "hip"):
    if name not in _IMPLEMENTATIONS:
        raise NotImplementedError(f"scan implementation {name!r} is not compiled (available: hip)")
    return _IMPLEMENTATIONS[name]
