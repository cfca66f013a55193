"""Input pytree types of the learner, mirroring boonta/utils/timestep.py:9-37
(``Timestep``) and boonta/utils/transition.py:10-26 (``Transition``).

Leaves are device tensors in the rollout's time-major layout [T, N, ...];
``terminated``/``truncated`` are bool (one byte per flag).
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True)
class Timestep:
    obs: Any
    action: Any = None
    reward: Any = None
    terminated: Any = None
    truncated: Any = None
    info: Any = None

    @property
    def done(self):
        """terminated OR truncated (timestep.py:17-19)."""
        return self.terminated | self.truncated

    def replace(self, **kw) -> "Timestep":
        return dataclasses.replace(self, **kw)


@dataclass(frozen=True)
class Transition:
    first: Timestep | None = None
    second: Timestep | None = None
    aux: dict | None = None
    carry: Any = None

    @property
    def start(self):
        """carry[0] (transition.py:16-18)."""
        return None if self.carry is None else self.carry[0]

    def replace(self, **kw) -> "Transition":
        return dataclasses.replace(self, **kw)
