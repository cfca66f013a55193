from .advantage_estimators import generalized_advantage_estimator
from .ppo import PPO, PPOConfig, PPOState

__all__ = ["PPO", "PPOConfig", "PPOState", "generalized_advantage_estimator"]
