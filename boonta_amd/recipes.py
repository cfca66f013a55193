"""The five learner workloads, composed the way boonta's recipes compose them
(hangar/recipes/ppo_cartpole.py:24-48, recurrent_ppo_classic_control.py:71-120,
recurrent_ppo_minatar.py:168-220), with the PPO defaults of
hangar/config/algorithm/{ppo,recurrent_ppo}.yaml and the optimizer chain
``chain(clip_by_global_norm(0.5), adam(lr))`` every PPO recipe builds.

  1  discrete, tiny:   obs [128, 4, 4];        2 actions; separate 2x64 tanh (orthogonal)
  2  discrete, Anakin: obs [128, 2048, 400];   6 actions; shared 2x256 ReLU
  3  Gaussian:         obs [16, 4096, 87];     D = 8, state-independent scale; separate 4x256 LN+SiLU
  4  recurrent GRU:    obs [64, 1024, 128];    8 actions; Dense256+ReLU -> GRU(256)
  5  large obs, bf16:  obs [64, 1024, 8268];   43 actions; shared 3x512 LN+ReLU
  6  RecurrentPuPO:    workload 4's rollout and network under RecurrentPuPO
                       (hangar/config/algorithm/recurrent_pupo.yaml: advantage and trace
                       clip 1, priority exponent 0.8, minibatch advantages normalised,
                       importance exponent 0.2), 4 epochs x 4 draws of 256 envs
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from . import networks as nn
from . import optim
from .algorithms.ppo import PPOConfig
from .algorithms.recurrent_pupo import RecurrentPuPOConfig


@dataclass(frozen=True)
class Recipe:
    name: str
    network: nn.Network
    cfg: PPOConfig
    optimizer: optim.Chain
    T: int
    N: int
    obs_dim: int
    seed: int
    done_p: float
    recurrent: bool = False
    algorithm: str = "ppo"   # "ppo" (PPO / RecurrentPPO) or "pupo" (RecurrentPuPO)

    @property
    def batch(self) -> int:
        return self.T * self.N

    @property
    def minibatch(self) -> int:
        n = self.N if self.recurrent else self.T * self.N
        return n // self.cfg.num_minibatches

    def resized(self, T: int | None = None, N: int | None = None, num_minibatches: int | None = None,
                update_epochs: int | None = None) -> "Recipe":
        """Same network and hyper-parameters on a smaller rollout (parity tests)."""
        cfg = self.cfg
        if num_minibatches is not None or update_epochs is not None:
            cfg = replace(cfg, num_minibatches=num_minibatches or cfg.num_minibatches,
                          update_epochs=update_epochs or cfg.update_epochs)
        return replace(self, T=T or self.T, N=N or self.N, cfg=cfg)


def _cfg(num_minibatches, update_epochs=4, clip=0.2, gamma=0.99, lam=0.95):
    return PPOConfig(num_minibatches=num_minibatches, update_epochs=update_epochs, clip_coefficient=clip,
                     clip_value_loss=True, entropy_coefficient=0.01, value_coefficient=0.5, gamma=gamma,
                     gae_lambda=lam, normalize_advantage=False)


def _opt(lr, max_grad_norm=0.5):
    return optim.chain(optim.clip_by_global_norm(max_grad_norm), optim.adam(lr))


def config1() -> Recipe:
    o = nn.orthogonal
    actor = nn.Categorical(nn.Sequential([
        nn.Dense(64, kernel_init=o(np.sqrt(2))), nn.tanh,
        nn.Dense(64, kernel_init=o(np.sqrt(2))), nn.tanh,
        nn.Dense(2, kernel_init=o(0.01))]))
    critic = nn.Sequential([
        nn.Dense(64, kernel_init=o(np.sqrt(2))), nn.tanh,
        nn.Dense(64, kernel_init=o(np.sqrt(2))), nn.tanh,
        nn.Dense(1, kernel_init=o(1.0))])
    net = nn.Network(feature_extractor=nn.FeatureExtractor(nn.Identity()),
                     head=nn.ActorCritic(actor=actor, critic=critic))
    return Recipe("discrete-tiny", net, _cfg(4), _opt(2.5e-4), T=128, N=4, obs_dim=4, seed=1001, done_p=0.01)


def config2() -> Recipe:
    net = nn.Network(
        feature_extractor=nn.FeatureExtractor(nn.Sequential([nn.Dense(256), nn.relu, nn.Dense(256), nn.relu])),
        head=nn.ActorCritic(actor=nn.Categorical(nn.Dense(6)), critic=nn.Dense(1)))
    return Recipe("discrete-anakin", net, _cfg(8), _opt(3e-4), T=128, N=2048, obs_dim=400, seed=1002,
                  done_p=0.005)


def _ln_silu_tower(width=256, depth=4):
    layers = []
    for _ in range(depth):
        layers += [nn.Dense(width), nn.LayerNorm(), nn.silu]
    return layers


def config3() -> Recipe:
    actor = nn.Gaussian(nn.Sequential(_ln_silu_tower() + [nn.SpreadScale(8)]))
    critic = nn.Sequential(_ln_silu_tower() + [nn.Dense(1)])
    net = nn.Network(feature_extractor=nn.FeatureExtractor(nn.Identity()),
                     head=nn.ActorCritic(actor=actor, critic=critic))
    return Recipe("gaussian", net, _cfg(32, clip=0.3, gamma=0.97), _opt(3e-4), T=16, N=4096, obs_dim=87,
                  seed=1003, done_p=0.001)


def config4() -> Recipe:
    net = nn.Network(
        feature_extractor=nn.FeatureExtractor(nn.Sequential([nn.Dense(256), nn.relu])),
        torso=nn.RNN(nn.GRUCell(256)),
        head=nn.ActorCritic(actor=nn.Categorical(nn.Dense(8)), critic=nn.Dense(1)))
    return Recipe("recurrent-gru", net, _cfg(4), _opt(2.5e-4), T=64, N=1024, obs_dim=128, seed=1004,
                  done_p=0.02, recurrent=True)


def config5() -> Recipe:
    bf = "bfloat16"
    layers = []
    for _ in range(3):
        layers += [nn.Dense(512, dtype=bf), nn.LayerNorm(dtype=bf), nn.relu]
    net = nn.Network(
        feature_extractor=nn.FeatureExtractor(nn.Sequential(layers)),
        head=nn.ActorCritic(actor=nn.Categorical(nn.Dense(43, dtype=bf)), critic=nn.Dense(1, dtype=bf)))
    return Recipe("large-obs-bf16", net, _cfg(8, lam=0.8), _opt(3e-4), T=64, N=1024, obs_dim=8268, seed=1005,
                  done_p=0.002)


def config6() -> Recipe:
    r = config4()
    c = r.cfg
    cfg = RecurrentPuPOConfig(num_minibatches=c.num_minibatches, update_epochs=c.update_epochs,
                              clip_coefficient=c.clip_coefficient, clip_value_loss=c.clip_value_loss,
                              entropy_coefficient=c.entropy_coefficient, value_coefficient=c.value_coefficient,
                              gamma=c.gamma, gae_lambda=c.gae_lambda)
    return replace(r, name="recurrent-pupo", cfg=cfg, seed=1006, algorithm="pupo")


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5, 6: config6}


def make(config: int) -> Recipe:
    return CONFIGS[int(config)]()
