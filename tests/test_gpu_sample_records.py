"""The fused loss's per-sample inputs (log_prob, value, advantage, return,
categorical action; the gathers of boonta/algorithms/ppo.py:148-151) read from
one 32-byte record per sample (ppo_pack_samples, sample_stride 8) against the
separate columns: the same values, so the parameters and logs of two whole
updates are the same bits.  The discrete workload at its full 32768-row
minibatch (the 64-row-tile head kernel), the Gaussian towers (the forward
chain that runs the heads + loss) and the GRU learner."""
import numpy as np
import pytest
import torch

from boonta_amd.algorithms import PPO, RecurrentPPO
from boonta_amd.algorithms.ppo import flat_state_of
from boonta_amd.random import key as make_key
from ppo_cases import device_recurrent_transition, device_transition, make_case, make_recurrent_case

pytestmark = pytest.mark.gpu

CASES = {"discrete": (PPO, 2, 16, 2048, 1, 2), "gaussian": (PPO, 3, 8, 250, 4, 2),
         "gru": (RecurrentPPO, 4, 16, 256, 4, 2)}


def columns(alg_cls):
    ex_cls = alg_cls.executor_class
    return type("Columns" + alg_cls.__name__, (alg_cls,),
                {"executor_class": type("Columns" + ex_cls.__name__, (ex_cls,), {"RECORDS": False})})


def run(alg_cls, config, T, N, M, E):
    if not issubclass(alg_cls, RecurrentPPO):
        r, plan, params, tr, roll = make_case(config=config, T=T, N=N, M=M, E=E)
        trans = device_transition(tr, roll)
    else:
        r, plan, params, tr, roll, extra = make_recurrent_case(config, T=T, N=N, M=M, E=E, seed=3)
        trans = device_recurrent_transition(tr, roll, extra)
    alg = alg_cls(cfg=r.cfg, network=r.network, optimizer=r.optimizer, use_graph=True)
    state = alg.init_from_params({"params": params}, r.obs_dim)
    ex = alg.executor(state, r.T, r.N, r.obs_dim)
    for k in (1, 2):
        alg.update(state, make_key(k), trans)
    torch.cuda.synchronize()
    return ex, flat_state_of(state).P.cpu().numpy().copy(), ex.LOGS.cpu().numpy().copy()


@pytest.mark.parametrize("name", sorted(CASES))
def test_records_give_the_bits_of_separate_columns(name):
    alg_cls, config, T, N, M, E = CASES[name]
    print(f"sample records case={name}", flush=True)
    ex_r, p_r, logs_r = run(alg_cls, config, T, N, M, E)
    ex_c, p_c, logs_c = run(columns(alg_cls), config, T, N, M, E)
    assert ex_r.REC is not None and ex_r._sample_stride() == 8 and ex_c.REC is None
    np.testing.assert_array_equal(p_r, p_c)
    np.testing.assert_array_equal(logs_r, logs_c)
    assert np.isfinite(logs_r).all()
