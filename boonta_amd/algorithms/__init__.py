from .advantage_estimators import generalized_advantage_estimator
from .ppo import PPO, PPOConfig, PPOState
from .recurrent_ppo import RecurrentPPO, RecurrentPPOConfig, RecurrentPPOState

__all__ = ["PPO", "PPOConfig", "PPOState", "RecurrentPPO", "RecurrentPPOConfig", "RecurrentPPOState",
           "generalized_advantage_estimator"]
