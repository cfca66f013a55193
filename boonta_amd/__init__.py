"""boonta_amd: boonta's PPO learner update (GAE, actor-critic forward and
backward, fused PPO loss, clip + Adam) as hand-written HIP kernels for MI355X
(gfx950), behind boonta's PPO / RecurrentPPO algorithm interface.

The kernels live in ``libppo_hip.so`` (C ABI: include/ppo_hip.h), built from
``boonta_amd/csrc``; there is no CPU or PyTorch fallback.
"""
from . import networks, optim, random
from .types import Timestep, Transition

__all__ = ["networks", "optim", "random", "Timestep", "Transition"]
