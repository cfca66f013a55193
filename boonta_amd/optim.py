"""Optimizer description for the learner: the optax chain every boonta PPO
recipe builds, ``optax.chain(optax.clip_by_global_norm(max_grad_norm),
optax.adam(lr))`` (hangar/recipes/ppo_cartpole.py:44-47), with optax 0.2.8's
state layout so a PPOState keeps the reference's tree shape:

    (EmptyState(), (ScaleByAdamState(count, mu, nu), EmptyState()))

The update itself runs in the fused HIP kernel ``ppo_adam_clip_f32``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, NamedTuple


@dataclass(frozen=True)
class ClipByGlobalNorm:
    max_norm: float


@dataclass(frozen=True)
class Adam:
    learning_rate: float
    b1: float = 0.9
    b2: float = 0.999
    eps: float = 1e-8
    eps_root: float = 0.0


@dataclass(frozen=True)
class Chain:
    transforms: tuple

    @property
    def max_grad_norm(self) -> float | None:
        for t in self.transforms:
            if isinstance(t, ClipByGlobalNorm):
                return t.max_norm
        return None

    @property
    def adam(self) -> Adam:
        for t in self.transforms:
            if isinstance(t, Adam):
                return t
        raise NotImplementedError("the learner compiles chains ending in adam")


def clip_by_global_norm(max_norm: float) -> ClipByGlobalNorm:
    return ClipByGlobalNorm(float(max_norm))


def adam(learning_rate: float, b1: float = 0.9, b2: float = 0.999, eps: float = 1e-8,
         eps_root: float = 0.0) -> Adam:
    if eps_root != 0.0:
        raise NotImplementedError("eps_root != 0 is not compiled")
    return Adam(float(learning_rate), float(b1), float(b2), float(eps), float(eps_root))


def chain(*transforms) -> Chain:
    kinds = [type(t) for t in transforms]
    if kinds not in ([ClipByGlobalNorm, Adam], [Adam]):
        raise NotImplementedError("the learner compiles chain(clip_by_global_norm, adam) or adam")
    return Chain(tuple(transforms))


class EmptyState(NamedTuple):
    pass


class ScaleByAdamState(NamedTuple):
    count: Any  # int32 scalar (device)
    mu: Any     # parameter tree
    nu: Any


def as_chain(opt) -> Chain:
    if isinstance(opt, Chain):
        return opt
    if isinstance(opt, Adam):
        return Chain((opt,))
    raise NotImplementedError(f"optimizer {opt!r} is not compiled")


@dataclass(frozen=True)
class ConstantSchedule:
    """optax.constant_schedule(value): the same value at every step."""
    value: float

    def __call__(self, step) -> float:
        return self.value


def constant_schedule(value: float) -> ConstantSchedule:
    return ConstantSchedule(float(value))
