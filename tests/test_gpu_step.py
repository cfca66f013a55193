"""Parity of the rollout-side PPO.step (boonta/algorithms/ppo.py:57-74) and
its sampling kernels against the oracle (oracle/sample.py, oracle/nets.py) on
the same seeded inputs, and the replay invariant of the reference's
tests/test_algorithms.py:343-366: an update whose optimizer does not move the
parameters recomputes exactly the log-probabilities its rollout acted on.

Tolerances (written here):
- sampled categorical actions bit-exact wherever the oracle's two largest
  perturbed logits differ by more than 1e-4 (fp32; 2e-2, about two bf16
  rounding steps of a unit logit, for the bf16 network), and at least 90 % of
  rows must qualify;
- log-probabilities and values 1e-5 relative (atol 1e-5) in fp32, 2e-2 for
  the bf16 network;
- Gaussian actions 1e-5 relative to |sigma eps| + |mean| (atol 1e-6): the
  float32 erfinv (Giles' polynomial) against scipy's float64 erfinv;
- replay: |approximate KL| <= 1e-6 and clip fraction 0 in every step.
"""
import numpy as np
import pytest
import torch

import synthetic
from boonta_amd import _lib, optim, recipes
from boonta_amd.algorithms.ppo import PPO, flat_state_of
from boonta_amd.random import key as make_key
from boonta_amd.types import Timestep, Transition
from oracle import nets, sample
from boonta_amd.algorithms.recurrent_ppo import RecurrentPPO
from ppo_cases import gpu_algorithm, gpu_recurrent_algorithm

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stream():
    return torch.cuda.current_stream().cuda_stream


def key_dev(k):
    return dev(np.asarray(k, np.uint32).view(np.int32))


def log_softmax64(x):
    x = np.asarray(x, np.float64)
    s = x - x.max(-1, keepdims=True)
    return s - np.log(np.exp(s).sum(-1, keepdims=True))


def check_categorical(act, lp, pref, key, temperature, margin_tol, rtol):
    a_or, _, margin = sample.categorical_sample(pref, key, temperature)
    ok = margin > margin_tol
    assert ok.mean() > 0.9
    np.testing.assert_array_equal(act[ok], a_or[ok])
    assert act.min() >= 0 and act.max() < pref.shape[1]
    rows = np.arange(len(act))
    if temperature > 0:
        want = log_softmax64(np.asarray(pref, np.float64) / temperature)[rows, act]
    else:
        want = np.where(act == np.argmax(pref, -1), 0.0, -np.inf)
    np.testing.assert_allclose(lp, want, rtol=rtol, atol=rtol)


@pytest.mark.parametrize("A", [1, 2, 6, 43, 128])
@pytest.mark.parametrize("temperature", [1.0, 0.5, 0.0])
def test_categorical_kernel_matches_the_oracle(A, temperature):
    rng = np.random.default_rng(A)
    rows, ld = 1000, A + 3
    buf = rng.standard_normal((rows, ld)).astype(np.float32) * 2
    pref = buf[:, :A]
    key = make_key(31 + A)
    d = dev(buf)
    act = torch.empty(rows, dtype=torch.int32, device="cuda")
    lp = torch.empty(rows, dtype=torch.float32, device="cuda")
    val = torch.empty(rows, dtype=torch.float32, device="cuda")
    _lib.call("ppo_sample_categorical_f32", stream(), d.data_ptr(), ld, rows, A, d.data_ptr() + 4 * A, ld,
              key_dev(key).data_ptr(), temperature, act.data_ptr(), lp.data_ptr(), val.data_ptr())
    torch.cuda.synchronize()
    check_categorical(act.cpu().numpy(), lp.cpu().numpy(), pref, key, temperature, 1e-4, 1e-5)
    np.testing.assert_array_equal(val.cpu().numpy(), buf[:, A])


@pytest.mark.parametrize("D", [1, 8, 17])
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("temperature", [1.0, 0.5])
def test_gaussian_kernel_matches_the_oracle(D, per_row, temperature):
    rng = np.random.default_rng(100 + D)
    rows, ld = 3000, 2 * D + 1
    buf = rng.standard_normal((rows, ld)).astype(np.float32)
    vec = rng.standard_normal(D).astype(np.float32)
    mean = buf[:, :D]
    raw = buf[:, D:2 * D] if per_row else vec
    key = make_key(7 * D + int(per_row))
    d, v = dev(buf), dev(vec)
    act = torch.empty(rows, D, dtype=torch.float32, device="cuda")
    lp = torch.empty(rows, dtype=torch.float32, device="cuda")
    val = torch.empty(rows, dtype=torch.float32, device="cuda")
    scale, lds = (d.data_ptr() + 4 * D, ld) if per_row else (v.data_ptr(), 0)
    _lib.call("ppo_sample_gaussian_f32", stream(), d.data_ptr(), ld, scale, lds, rows, D, d.data_ptr() + 8 * D,
              ld, key_dev(key).data_ptr(), temperature, act.data_ptr(), D, lp.data_ptr(), val.data_ptr())
    torch.cuda.synchronize()
    a_or, lp_or, eps = sample.gaussian_sample(mean, raw, key, temperature)
    sig = temperature * (sample.softplus(np.broadcast_to(raw, mean.shape)) + 1e-3)
    a = act.cpu().numpy()
    np.testing.assert_array_less(np.abs(a - a_or), 1e-5 * (np.abs(sig * eps) + np.abs(mean)) + 1e-6)
    np.testing.assert_allclose(lp.cpu().numpy(), lp_or, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(val.cpu().numpy(), buf[:, 2 * D])


STEP_CASES = {
    "c1-tiny": dict(config=1, N=64),
    "c2-anakin": dict(config=2, N=512),
    "c3-gaussian": dict(config=3, N=512),
    "c5-bf16": dict(config=5, N=512),
}


@pytest.mark.parametrize("name", list(STEP_CASES))
@pytest.mark.parametrize("temperature", [1.0, 0.5])
def test_step_matches_the_oracle(name, temperature):
    case = STEP_CASES[name]
    r = recipes.make(case["config"]).resized(N=case["N"])
    N, D = r.N, r.obs_dim
    plan = r.network.plan(D)
    params = r.network.init(0, D)["params"]
    obs = synthetic.rollout(r, T=1, N=N)["obs"][0]
    head, value, _ = nets.forward(params, plan, obs)
    alg = gpu_algorithm(r, use_graph=False)
    state = alg.init_from_params({"params": params}, D)
    key = make_key(2024)
    _, carry, action, aux = alg.step(state, None, key, Timestep(obs=dev(obs)), temperature=temperature)
    torch.cuda.synchronize()
    assert carry is None
    bf16 = plan.get("compute_dtype") == "bfloat16"
    rtol = 2e-2 if bf16 else 1e-5
    np.testing.assert_allclose(aux["value"].cpu().numpy(), value, rtol=rtol, atol=rtol)
    dist = plan["dist"]
    if dist["kind"] == "categorical":
        check_categorical(action.cpu().numpy(), aux["log_prob"].cpu().numpy(), head, key, temperature,
                          2e-2 if bf16 else 1e-4, rtol)
    else:
        Dm = dist["dim"]
        if dist.get("scale") is not None:
            mean, raw = head, np.asarray(nets.get(params, dist["scale"]), np.float64)
        else:
            mean, raw = head[:, :Dm], head[:, Dm:]
        a_or, lp_or, eps = sample.gaussian_sample(mean, raw, key, temperature)
        sig = temperature * (sample.softplus(np.broadcast_to(raw, mean.shape)) + 1e-3)
        a = action.cpu().numpy()
        assert a.shape == (N, Dm)
        np.testing.assert_array_less(np.abs(a - a_or), 1e-5 * (np.abs(sig * eps) + np.abs(mean)) + 1e-5)
        np.testing.assert_allclose(aux["log_prob"].cpu().numpy(), lp_or, rtol=rtol, atol=rtol)


@pytest.mark.parametrize("rows,pad,temperature", [(1000, 1, 1.0), (2048, 0, 0.7), (37, 3, 0.0)])
def test_one_launch_step_matches_the_oracle_and_the_chained_launches(rows, pad, temperature):
    """The discrete Anakin network's whole step in one launch
    (ppo_step_mlp_categorical_f32): ragged row counts, observation rows with
    and without 16-byte pitch (pad extra floats per row), greedy draws; against
    the oracle and the layer-by-layer launches on the same inputs."""
    from boonta_amd.rollout import StepExecutor
    r = recipes.make(2).resized(N=rows)
    D = r.obs_dim
    params = r.network.init(5, D)["params"]
    obs = synthetic.rollout(r, T=1, N=rows)["obs"][0]
    head, value, _ = nets.forward(params, r.network.plan(D), obs)
    alg = gpu_algorithm(r, use_graph=False)
    state = alg.init_from_params({"params": params}, D)
    prog = alg.program(D)
    o = torch.zeros(rows, D + pad, device="cuda")
    o[:, :D] = dev(obs)
    key = make_key(77)
    out = {}
    for fused in (True, False):
        ex = StepExecutor(prog, flat_state_of(state), rows, fused=fused)
        assert ex.fused == fused
        ex.KEY.copy_(key_dev(key))
        act = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
        lp = torch.full((rows,), float("nan"), device="cuda")
        v = torch.full((rows,), float("nan"), device="cuda")
        ex.issue(stream(), o.data_ptr(), D + pad, temperature, act.data_ptr(), lp.data_ptr(), v.data_ptr())
        torch.cuda.synchronize()
        out[fused] = (act.cpu().numpy(), lp.cpu().numpy(), v.cpu().numpy())
    act, lp, v = out[True]
    np.testing.assert_allclose(v, value, rtol=1e-5, atol=1e-5)
    check_categorical(act, lp, head, key, temperature, 1e-4, 1e-5)
    np.testing.assert_allclose(v, out[False][2], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(lp, out[False][1], rtol=1e-5, atol=1e-5)
    assert (act == out[False][0]).mean() > 0.99


FUSED_NETS = [
    # (trunk layers, activation, actions, observation features, row padding)
    (1, "tanh", 2, 3, 1),        # narrowest observation, one layer
    (3, "silu", 15, 60, 0),      # widest head (16-column kernel), obs width not a multiple of 16
    (4, None, 15, 1023, 1),      # deepest trunk, no activation, 1023 features on 16-byte rows
    (4, "tanh", 2, 1024, 0),     # the widest observation the LDS stage holds
    (3, None, 2, 1024, 0),
    (1, "silu", 15, 1023, 0),    # 1023 features on rows without 16-byte pitch
    (2, "tanh", 7, 64, 3),
]


@pytest.mark.parametrize("layers,act,A,D,pad", FUSED_NETS)
def test_one_launch_step_on_every_network_it_accepts(layers, act, A, D, pad):
    """Every shared-trunk float32 network the one-launch step takes (1-4
    layers of 256 features with one activation or none, at most 15 actions,
    at most ppo_step_mlp_max_obs() observation features): the fused step
    against the oracle's forward and categorical draw, and against the
    layer-by-layer launches, on 300 rows (ragged against the 16-row tiles)."""
    from boonta_amd import networks as nn
    from boonta_amd.rollout import StepExecutor
    rows = 300
    trunk = []
    for _ in range(layers):
        trunk.append(nn.Dense(256))
        if act is not None:
            trunk.append({"tanh": nn.tanh, "silu": nn.silu}[act])
    net = nn.Network(feature_extractor=nn.FeatureExtractor(nn.Sequential(trunk)),
                     head=nn.ActorCritic(actor=nn.Categorical(nn.Dense(A)), critic=nn.Dense(1)))
    params = net.init(layers * 100 + A, D)["params"]
    rng = np.random.default_rng(D + A)
    obs = rng.standard_normal((rows, D)).astype(np.float32)
    head, value, _ = nets.forward(params, net.plan(D), obs)
    alg = PPO(cfg=recipes.make(2).cfg, network=net, optimizer=recipes.make(2).optimizer, use_graph=False)
    state = alg.init_from_params({"params": params}, D)
    prog = alg.program(D)
    o = torch.zeros(rows, D + pad, device="cuda")
    o[:, :D] = dev(obs)
    key = make_key(layers + 10 * A)
    out = {}
    for fused in (True, False):
        ex = StepExecutor(prog, flat_state_of(state), rows, fused=fused)
        assert ex.fused == fused
        ex.KEY.copy_(key_dev(key))
        a_ = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
        lp = torch.full((rows,), float("nan"), device="cuda")
        v = torch.full((rows,), float("nan"), device="cuda")
        ex.issue(stream(), o.data_ptr(), D + pad, 1.0, a_.data_ptr(), lp.data_ptr(), v.data_ptr())
        torch.cuda.synchronize()
        out[fused] = (a_.cpu().numpy(), lp.cpu().numpy(), v.cpu().numpy())
    a_, lp, v = out[True]
    np.testing.assert_allclose(v, value, rtol=1e-5, atol=1e-5)
    check_categorical(a_, lp, head, key, 1.0, 1e-4, 1e-5)
    np.testing.assert_allclose(v, out[False][2], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(lp, out[False][1], rtol=1e-5, atol=1e-5)
    assert (a_ == out[False][0]).mean() > 0.99


def test_one_launch_step_replays_from_a_graph():
    """The rollout bench captures env steps into a HIP graph: every replay,
    with eager work and synchronisations between replays, equals the eager
    step bit for bit."""
    from boonta_amd.rollout import StepExecutor
    rows = 2048
    r = recipes.make(2).resized(N=rows)
    D = r.obs_dim
    params = r.network.init(8, D)["params"]
    obs = dev(synthetic.rollout(r, T=1, N=rows)["obs"][0])
    alg = gpu_algorithm(r, use_graph=False)
    state = alg.init_from_params({"params": params}, D)
    ex = StepExecutor(alg.program(D), flat_state_of(state), rows)
    assert ex.fused
    ex.KEY.copy_(key_dev(make_key(31)))
    act = torch.zeros(rows, dtype=torch.int32, device="cuda")
    lp = torch.zeros(rows, device="cuda")
    v = torch.zeros(rows, device="cuda")
    args = (obs.data_ptr(), D, 1.0, act.data_ptr(), lp.data_ptr(), v.data_ptr())
    ex.issue(stream(), *args)
    torch.cuda.synchronize()
    want = (act.clone(), lp.clone(), v.clone())
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            ex.issue(side.cuda_stream, *args)
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(3):
        act.fill_(-1)
        lp.zero_()
        v.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(act, want[0]) and torch.equal(lp, want[1]) and torch.equal(v, want[2])


def test_step_takes_a_device_key_and_follows_the_updated_parameters():
    r = recipes.make(2).resized(N=256)
    D = r.obs_dim
    params = r.network.init(3, D)["params"]
    obs = synthetic.rollout(r, T=1, N=r.N)["obs"][0]
    alg = gpu_algorithm(r, use_graph=False)
    state = alg.init_from_params({"params": params}, D)
    key = make_key(9)
    o = dev(obs)
    _, _, a1, x1 = alg.step(state, None, key, Timestep(obs=o))
    _, _, a2, x2 = alg.step(state, None, key_dev(key), Timestep(obs=o))
    torch.cuda.synchronize()
    assert torch.equal(a1, a2) and torch.equal(x1["log_prob"], x2["log_prob"])
    # parameters changed in place are seen by the next step (one flat buffer)
    flat_state_of(state).P.add_(0.01)
    _, _, a3, x3 = alg.step(state, None, key, Timestep(obs=o))
    torch.cuda.synchronize()
    assert not torch.equal(x1["value"], x3["value"])


@pytest.mark.parametrize("config", [1, 2, 3])
def test_update_replays_what_step_acted_on(config):
    """tests/test_algorithms.py:343-366: with an optimizer that leaves the
    parameters where they are, every minibatch's recomputed log-probabilities
    equal the rollout's (KL 0, nothing clipped)."""
    r = recipes.make(config).resized(T=8, N=64, num_minibatches=4, update_epochs=2)
    T, N, D = r.T, r.N, r.obs_dim
    roll = synthetic.rollout(r, T, N)
    alg = PPO(cfg=r.cfg, network=r.network, optimizer=optim.chain(optim.clip_by_global_norm(0.5), optim.adam(0.0)))
    obs = dev(roll["obs"])
    state, _ = alg.init(make_key(0), Timestep(obs=obs[0]))
    actions, lps, values = [], [], []
    for t in range(T):
        _, _, a, aux = alg.step(state, None, make_key(100 + t), Timestep(obs=obs[t].contiguous()))
        actions.append(a)
        lps.append(aux["log_prob"])
        values.append(aux["value"])
    second = Timestep(obs=obs[1:], action=torch.stack(actions), reward=dev(roll["reward"]),
                      terminated=dev(roll["terminated"]), truncated=dev(roll["truncated"]))
    trans = Transition(first=Timestep(obs=obs[:-1]), second=second,
                       aux={"log_prob": torch.stack(lps), "value": torch.stack(values)})
    alg.update(state, make_key(5), trans)
    torch.cuda.synchronize()
    logs = alg.logs(state, T, N, D)
    assert np.all(np.abs(logs["actor/approximate_kl"]) <= 1e-6), logs["actor/approximate_kl"]
    np.testing.assert_array_equal(logs["actor/clip_fraction"], 0.0)


def test_recurrent_step_matches_the_oracle():
    """RecurrentPPO.step (recurrent_ppo.py:71-96): reset where done, one GRU
    step, heads on the new carry, then the categorical draw."""
    r = recipes.make(4).resized(N=256)
    N, D = r.N, r.obs_dim
    plan = r.network.plan(D)
    H = plan["torso"]["features"]
    params = r.network.init(0, D)["params"]
    rng = np.random.default_rng(4)
    obs = synthetic.rollout(r, T=1, N=N)["obs"][0]
    carry = np.tanh(rng.standard_normal((N, H))).astype(np.float32)
    term = rng.random(N) < 0.2
    trunc = (rng.random(N) < 0.1) & ~term
    head, value, final, _ = nets.recurrent_forward(params, plan, obs[:, None, :], (term | trunc)[:, None], carry)
    alg = gpu_recurrent_algorithm(r, use_graph=False)
    state = alg.init_from_params({"params": params}, D)
    key = make_key(44)
    _, c2, action, aux = alg.step(state, dev(carry), key, Timestep(obs=dev(obs), terminated=dev(term),
                                                                    truncated=dev(trunc)))
    torch.cuda.synchronize()
    np.testing.assert_allclose(c2.cpu().numpy(), final, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(aux["value"].cpu().numpy(), value[:, 0], rtol=1e-5, atol=1e-5)
    check_categorical(action.cpu().numpy(), aux["log_prob"].cpu().numpy(), head[:, 0], key, 1.0, 1e-4, 1e-5)
    # no carry is the zero carry; with every env done the given carry is forgotten
    _, c0, a0, x0 = alg.step(state, None, key, Timestep(obs=dev(obs)))
    done = torch.ones(N, dtype=torch.bool, device="cuda")
    _, c1, a1, x1 = alg.step(state, dev(carry), key, Timestep(obs=dev(obs), terminated=done,
                                                                truncated=torch.zeros_like(done)))
    torch.cuda.synchronize()
    assert torch.equal(c0, c1) and torch.equal(a0, a1) and torch.equal(x0["log_prob"], x1["log_prob"])


def test_recurrent_update_replays_what_step_acted_on():
    """tests/test_algorithms.py:368-380 (every torso replays what it acted
    on): the update's sequence minibatches recompute the step-by-step GRU from
    carry[0] with the resets first.done."""
    r = recipes.make(4).resized(T=8, N=64, num_minibatches=4, update_epochs=2)
    T, N, D = r.T, r.N, r.obs_dim
    roll = synthetic.rollout(r, T, N)
    first_term = np.concatenate([roll["first_done"][:1], roll["terminated"][:-1]], axis=0)
    first_trunc = np.concatenate([np.zeros((1, N), bool), roll["truncated"][:-1]], axis=0)
    alg = RecurrentPPO(cfg=r.cfg, network=r.network,
                       optimizer=optim.chain(optim.clip_by_global_norm(0.5), optim.adam(0.0)))
    obs = dev(roll["obs"])
    state, carry = alg.init(make_key(0), Timestep(obs=obs[0]))
    carry = torch.tanh(torch.randn(carry.shape, generator=torch.Generator().manual_seed(3))).cuda()
    ft, ftr = dev(first_term), dev(first_trunc)
    carries, actions, lps, values = [], [], [], []
    for t in range(T):
        carries.append(carry)
        _, carry, a, aux = alg.step(state, carry, make_key(200 + t),
                                    Timestep(obs=obs[t].contiguous(), terminated=ft[t], truncated=ftr[t]))
        actions.append(a)
        lps.append(aux["log_prob"])
        values.append(aux["value"])
    second = Timestep(obs=obs[1:], action=torch.stack(actions), reward=dev(roll["reward"]),
                      terminated=dev(roll["terminated"]), truncated=dev(roll["truncated"]))
    trans = Transition(first=Timestep(obs=obs[:-1], terminated=ft, truncated=ftr), second=second,
                       aux={"log_prob": torch.stack(lps), "value": torch.stack(values)},
                       carry=torch.stack(carries))
    alg.update(state, make_key(5), trans)
    torch.cuda.synchronize()
    logs = alg.logs(state, T, N, D)
    assert np.all(np.abs(logs["actor/approximate_kl"]) <= 1e-6), logs["actor/approximate_kl"]
    np.testing.assert_array_equal(logs["actor/clip_fraction"], 0.0)
