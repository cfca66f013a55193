from .advantage_estimators import generalized_advantage_estimator
from .ppo import PPO, PPOConfig, PPOState
from .recurrent_ppo import RecurrenceError, RecurrentPPO, RecurrentPPOConfig, RecurrentPPOState
from .recurrent_pupo import RecurrentPuPO, RecurrentPuPOConfig, RecurrentPuPOState

__all__ = ["PPO", "PPOConfig", "PPOState", "RecurrentPPO", "RecurrentPPOConfig", "RecurrentPPOState",
           "RecurrentPuPO", "RecurrentPuPOConfig", "RecurrentPuPOState", "generalized_advantage_estimator"]
