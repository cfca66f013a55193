"""Pins the oracle's hand-written backward passes and the loss gradient with
float64 central finite differences of the scalar loss, on every network shape
the learner compiles (tanh / ReLU / LayerNorm + SiLU MLPs, Categorical and
Gaussian heads, shared and separate towers, the GRU torso), plus the
reference's torso invariants and the optimizer's closed forms."""
import copy

import numpy as np
import pytest

from boonta_amd import networks as nn
from boonta_amd import recipes
from oracle import nets, ppo

CFG = {"clip_coefficient": 0.2, "clip_value_loss": True, "entropy_coefficient": 0.01,
       "value_coefficient": 0.5}


def small_plans():
    o = nn.orthogonal
    sep_tanh = nn.Network(head=nn.ActorCritic(
        actor=nn.Categorical(nn.Sequential([nn.Dense(8, kernel_init=o(1.4)), nn.tanh, nn.Dense(3)])),
        critic=nn.Sequential([nn.Dense(8), nn.tanh, nn.Dense(1)])))
    shared_relu = nn.Network(
        feature_extractor=nn.FeatureExtractor(nn.Sequential([nn.Dense(8), nn.relu, nn.Dense(8), nn.relu])),
        head=nn.ActorCritic(actor=nn.Categorical(nn.Dense(4)), critic=nn.Dense(1)))
    ln_silu_gauss = nn.Network(head=nn.ActorCritic(
        actor=nn.Gaussian(nn.Sequential([nn.Dense(8), nn.LayerNorm(), nn.silu, nn.SpreadScale(2)])),
        critic=nn.Sequential([nn.Dense(8), nn.LayerNorm(), nn.silu, nn.Dense(1)])))
    gauss_state_dep = nn.Network(
        feature_extractor=nn.FeatureExtractor(nn.Sequential([nn.Dense(8), nn.tanh])),
        head=nn.ActorCritic(actor=nn.Gaussian(nn.Dense(4)), critic=nn.Dense(1)))
    return {"separate-tanh": sep_tanh, "shared-relu": shared_relu, "ln-silu-gaussian": ln_silu_gauss,
            "gaussian-state-dependent": gauss_state_dep}


def batch(plan, rng, rows, obs_dim):
    obs = rng.standard_normal((rows, obs_dim))
    d = plan["dist"]
    if d["kind"] == "categorical":
        action = rng.integers(0, d["num"], rows)
    else:
        action = rng.standard_normal((rows, d["dim"]))
    return dict(obs=obs, action=action, old_logp=rng.normal(-1.2, 0.3, rows),
                old_value=rng.normal(0, 1, rows), adv=rng.normal(0, 1, rows), ret=rng.normal(0, 1, rows))


def perturb(params, rng):
    # move LN scale/bias and the Gaussian scale off their init so their grads are generic
    def walk(t):
        for k, v in t.items():
            if isinstance(v, dict):
                walk(v)
            else:
                t[k] = np.asarray(v, np.float64) + 0.1 * rng.standard_normal(np.shape(v))
    walk(params)
    return params


def fd_check(loss_fn, params, grads, rng, picks=40, eps=1e-6):
    leaves = ppo.tree_leaves(params)
    gleaves = dict(ppo.tree_leaves(grads))
    checked = 0
    for _ in range(picks):
        path, leaf = leaves[rng.integers(len(leaves))]
        flat_i = rng.integers(np.size(leaf))
        p1, p2 = copy.deepcopy(params), copy.deepcopy(params)
        nets.get(p1, path[:-1])[path[-1]] = np.array(leaf, np.float64)
        nets.get(p2, path[:-1])[path[-1]] = np.array(leaf, np.float64)
        nets.get(p1, path[:-1])[path[-1]].reshape(-1)[flat_i] += eps
        nets.get(p2, path[:-1])[path[-1]].reshape(-1)[flat_i] -= eps
        fd = (loss_fn(p1) - loss_fn(p2)) / (2 * eps)
        an = np.asarray(gleaves[path]).reshape(-1)[flat_i]
        assert abs(fd - an) <= 1e-6 + 1e-5 * abs(fd), (path, flat_i, fd, an)
        checked += 1
    assert checked == picks


@pytest.mark.parametrize("name", list(small_plans()))
def test_mlp_loss_gradient_matches_finite_differences(name):
    net = small_plans()[name]
    rng = np.random.default_rng(hash(name) % 2**32)
    plan = net.plan(5)
    params = perturb(net.init(0, 5)["params"], rng)
    b = batch(plan, rng, 16, 5)

    def loss(p):
        return ppo.loss_and_grad(p, plan, CFG, b["obs"], b["action"], b["old_logp"], b["old_value"],
                                 b["adv"], b["ret"])[0]

    _, _, grads = ppo.loss_and_grad(params, plan, CFG, b["obs"], b["action"], b["old_logp"],
                                    b["old_value"], b["adv"], b["ret"])
    fd_check(loss, params, grads, rng)


def gru_net(H=6):
    return nn.Network(feature_extractor=nn.FeatureExtractor(nn.Sequential([nn.Dense(5), nn.relu])),
                      torso=nn.RNN(nn.GRUCell(H)),
                      head=nn.ActorCritic(actor=nn.Categorical(nn.Dense(3)), critic=nn.Dense(1)))


def test_gru_bptt_matches_finite_differences():
    rng = np.random.default_rng(4)
    net = gru_net()
    plan = net.plan(4)
    params = perturb(net.init(1, 4)["params"], rng)
    B, T = 3, 7
    obs = rng.standard_normal((B, T, 4))
    done = rng.random((B, T)) < 0.25
    carry = np.tanh(rng.standard_normal((B, 6)))
    act = rng.integers(0, 3, (B, T))
    olp, ov = rng.normal(-1.1, 0.3, (B, T)), rng.normal(0, 1, (B, T))
    adv, ret = rng.normal(0, 1, (B, T)), rng.normal(0, 1, (B, T))

    def run(p):
        return ppo.recurrent_loss_and_grad(p, plan, CFG, obs, done, carry, act, olp, ov, adv, ret)

    _, _, grads = run(params)
    fd_check(lambda p: run(p)[0], params, grads, rng, picks=60)


def test_gru_episode_start_forgets_the_past():
    # reference tests/test_networks.py:60-66
    rng = np.random.default_rng(5)
    net = gru_net()
    plan = net.plan(4)
    params = net.init(2, 4)["params"]
    B, T = 2, 9
    x = rng.standard_normal((B, T, 4))
    starts = np.zeros((B, T), bool)
    starts[:, 5] = True
    carry = np.tanh(rng.standard_normal((B, 6)))
    _, v1, _, _ = nets.recurrent_forward(params, plan, x, starts, carry)
    _, v2, _, _ = nets.recurrent_forward(params, plan, x[:, 5:], np.zeros((B, T - 5), bool), np.zeros((B, 6)))
    np.testing.assert_allclose(v1[:, 5:], v2, rtol=1e-12, atol=1e-12)


def test_gru_chunks_equal_steps():
    # reference tests/test_networks.py:51-57: a sequence in chunks == all at once
    rng = np.random.default_rng(6)
    net = gru_net()
    plan = net.plan(4)
    params = net.init(3, 4)["params"]
    x = rng.standard_normal((2, 8, 4))
    done = rng.random((2, 8)) < 0.3
    c0 = np.tanh(rng.standard_normal((2, 6)))
    _, full, _, _ = nets.recurrent_forward(params, plan, x, done, c0)
    _, a, c1, _ = nets.recurrent_forward(params, plan, x[:, :3], done[:, :3], c0)
    _, b, _, _ = nets.recurrent_forward(params, plan, x[:, 3:], done[:, 3:], c1)
    np.testing.assert_allclose(np.concatenate([a, b], 1), full, rtol=1e-12, atol=1e-12)


def test_replay_of_the_acting_policy_gives_ratio_one():
    # reference tests/test_algorithms.py:398-408: the first update replays the rollout's log-probs
    rng = np.random.default_rng(7)
    net = small_plans()["shared-relu"]
    plan = net.plan(5)
    params = net.init(4, 5)["params"]
    b = batch(plan, rng, 32, 5)
    logits, value, _ = nets.forward(params, plan, b["obs"])
    lp, _, _ = nets.categorical_stats(logits, b["action"])
    _, logs, _ = ppo.loss_and_grad(params, plan, CFG, b["obs"], b["action"], lp, value, b["adv"], b["ret"])
    assert abs(logs["actor/approximate_kl"]) < 1e-15
    assert logs["actor/clip_fraction"] == 0.0
    np.testing.assert_allclose(logs["actor/loss"], -b["adv"].mean(), rtol=1e-12)


def test_categorical_matches_log_softmax_and_entropy():
    rng = np.random.default_rng(8)
    z = rng.normal(0, 2, (50, 5))
    a = rng.integers(0, 5, 50)
    lp, ent, _ = nets.categorical_stats(z, a)
    ls = z - np.log(np.exp(z).sum(-1, keepdims=True))
    np.testing.assert_allclose(lp, ls[np.arange(50), a], rtol=1e-12)
    np.testing.assert_allclose(ent, -(np.exp(ls) * ls).sum(-1), rtol=1e-12)


def test_gaussian_matches_the_normal_density():
    rng = np.random.default_rng(9)
    mu, raw, x = rng.normal(size=(20, 3)), rng.normal(size=(20, 3)), rng.normal(size=(20, 3))
    sig = nets.gaussian_sigma(raw)
    np.testing.assert_allclose(sig, np.log1p(np.exp(raw)) + 1e-3, rtol=1e-12)
    lp, ent = nets.gaussian_stats(mu, sig, x)
    dens = np.prod(np.exp(-0.5 * ((x - mu) / sig) ** 2) / (sig * np.sqrt(2 * np.pi)), -1)
    np.testing.assert_allclose(lp, np.log(dens), rtol=1e-10)
    np.testing.assert_allclose(ent, (0.5 * np.log(2 * np.pi * np.e * sig ** 2)).sum(-1), rtol=1e-12)


def test_spread_scale_starts_at_unit_sigma():
    sc = nn.SpreadScale(3).scale_init
    np.testing.assert_allclose(nets.gaussian_sigma(np.float64(np.float32(sc))), 1.0, rtol=1e-6)


def test_adam_first_step_moves_each_weight_by_lr():
    rng = np.random.default_rng(10)
    p = {"w": rng.normal(size=50)}
    g = {"w": rng.normal(size=50)}
    new, st, _ = ppo.optimizer_update(g, ppo.optimizer_init(p), p, {"lr": 1e-3, "max_grad_norm": None})
    np.testing.assert_allclose(new["w"] - p["w"], -1e-3 * np.sign(g["w"]), rtol=1e-6)
    assert st["count"] == 1


def test_global_norm_clip_rescales_to_the_bound():
    rng = np.random.default_rng(11)
    g = {"a": rng.normal(size=10) * 10, "b": {"c": rng.normal(size=5) * 10}}
    p = ppo.tree_map(np.zeros_like, g)
    opt = {"lr": 1.0, "max_grad_norm": 0.5, "b1": 0.0, "b2": 0.0, "eps": 0.0}
    # with b1 = b2 = 0 and eps = 0 the step is g / |g| elementwise: clipping cannot be seen,
    # so check the clipped moments instead
    _, st, gn = ppo.optimizer_update(g, ppo.optimizer_init(p), p, opt)
    mu = np.concatenate([st["mu"]["a"], st["mu"]["b"]["c"]])
    np.testing.assert_allclose(np.linalg.norm(mu), 0.5, rtol=1e-12)
    assert gn > 0.5
    small = ppo.tree_map(lambda x: x * 1e-3, g)
    _, st2, _ = ppo.optimizer_update(small, ppo.optimizer_init(p), p, opt)
    np.testing.assert_allclose(st2["mu"]["a"], small["a"], rtol=1e-12)


@pytest.mark.parametrize("config", [1, 2, 3, 5])
def test_recipe_parameter_counts(config):
    # the parameter counts of the five workloads
    expected = {1: 9155, 2: 170247, 3: 446225, 5: 4784684}[config]
    r = recipes.make(config)
    params = r.network.init(0, r.obs_dim)["params"]
    assert sum(np.size(v) for _, v in ppo.tree_leaves(params)) == expected


def test_gru_recipe_parameter_count():
    r = recipes.make(4)
    params = r.network.init(0, r.obs_dim)["params"]
    assert sum(np.size(v) for _, v in ppo.tree_leaves(params)) == 429577


# ----------------------------------------------- pins against library routines
def _torch_gru_cell(params, H, I):
    """torch.nn.GRUCell in float64 holding flax GRUCell's parameters
    (boonta/networks/blocks/rnn.py:47-54): torch's gates are
    r = s(W_ir x + b_ir + W_hr h + b_hr), z = s(W_iz x + b_iz + W_hz h + b_hz),
    n = tanh(W_in x + b_in + r * (W_hn h + b_hn)), h' = (1 - z) n + z h; flax's
    recurrent r and z projections have no bias, so b_hr = b_hz = 0."""
    import torch
    cell = torch.nn.GRUCell(I, H).double()
    k = lambda n: torch.from_numpy(np.asarray(params[n]["kernel"], np.float64))
    b = lambda n: torch.from_numpy(np.asarray(params[n]["bias"], np.float64))
    with torch.no_grad():
        cell.weight_ih.copy_(torch.cat([k("ir"), k("iz"), k("in")], 1).T)
        cell.bias_ih.copy_(torch.cat([b("ir"), b("iz"), b("in")]))
        cell.weight_hh.copy_(torch.cat([k("hr"), k("hz"), k("hn")], 1).T)
        cell.bias_hh.copy_(torch.cat([torch.zeros(2 * H, dtype=torch.float64), b("hn")]))
    return cell


def test_gru_forward_matches_torch_grucell_with_resets():
    """The oracle's GRU recurrence against torch.nn.GRUCell stepped by hand
    over 12 steps, the carry zeroed before step t wherever done[b, t]
    (reset_carry, boonta/networks/blocks/rnn.py:11-16,42-45).  Every gate
    bias is moved off zero so that a swapped r / z pair or b_hn outside the
    reset gate changes the result."""
    import torch
    rng = np.random.default_rng(12)
    B, T, I, H = 5, 12, 7, 6
    net = nn.Network(torso=nn.RNN(nn.GRUCell(H)),
                     head=nn.ActorCritic(actor=nn.Categorical(nn.Dense(2)), critic=nn.Dense(1)))
    plan = net.plan(I)
    params = perturb(net.init(5, I)["params"], rng)
    torso = plan["torso"]
    gp = nets.get(params, torso["path"])
    for g in ("ir", "iz", "in", "hn"):
        gp[g]["bias"] = gp[g]["bias"] + rng.normal(0, 0.5, H)
    x = rng.standard_normal((B, T, I))
    done = rng.random((B, T)) < 0.2
    done[0, 4] = True
    carry = np.tanh(rng.standard_normal((B, H)))
    out, final, _ = nets.gru_forward(params, torso, x, done, carry)
    cell = _torch_gru_cell(gp, H, I)
    h = torch.from_numpy(carry)
    want = np.zeros((B, T, H))
    with torch.no_grad():
        for t in range(T):
            h = torch.where(torch.from_numpy(done[:, t:t + 1]), torch.zeros_like(h), h)
            h = cell(torch.from_numpy(x[:, t]), h)
            want[:, t] = h.numpy()
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(final, want[:, -1], rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("scale", [1.0, 1e-3])
def test_layernorm_forward_matches_torch_layer_norm(scale):
    """flax LayerNorm (epsilon 1e-6, scale and bias) against
    torch.nn.functional.layer_norm in float64.  At scale 1e-3 the row
    variance is about 1e-6, the size of epsilon, so a wrong epsilon, or
    epsilon applied outside the square root, is far outside the tolerance."""
    import torch
    rng = np.random.default_rng(13)
    F = 48
    x = scale * (rng.standard_normal((9, F)) + rng.normal(0, 3, (9, 1)))
    p = {"ln": {"scale": 1.0 + 0.2 * rng.standard_normal(F), "bias": 0.3 * rng.standard_normal(F)}}
    y, _ = nets.stages_forward(p, [{"op": "layernorm", "path": ("ln",), "eps": 1e-6}], x)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x), (F,), torch.from_numpy(p["ln"]["scale"]),
                                          torch.from_numpy(p["ln"]["bias"]), eps=1e-6).numpy()
    np.testing.assert_allclose(y, want, rtol=1e-9, atol=1e-9)


def test_adam_constant_gradient_moves_every_weight_by_lr_at_every_step():
    """With a constant gradient g the bias-corrected moments are exactly g and
    g^2 at every count t (mu_t = (1 - b1^t) g, nu_t = (1 - b2^t) g^2), so each
    step moves each weight by lr * |g| / (|g| + eps).  A bias correction taken
    at count - 1, or the decays swapped, breaks this from step 2 on."""
    rng = np.random.default_rng(14)
    p0 = {"w": rng.normal(size=40), "b": {"c": rng.normal(size=3)}}
    g = {"w": rng.normal(size=40) * 10.0 ** rng.integers(-3, 3, 40), "b": {"c": np.array([1e-2, -3.0, 0.5])}}
    opt = {"lr": 1e-3, "max_grad_norm": None}
    st = ppo.optimizer_init(p0)
    p = p0
    for t in range(1, 6):
        new, st, _ = ppo.optimizer_update(g, st, p, opt)
        assert st["count"] == t
        for path, gl in ppo.tree_leaves(g):
            step = nets.get(new, path[:-1])[path[-1]] - nets.get(p, path[:-1])[path[-1]]
            np.testing.assert_allclose(step, -1e-3 * gl / (np.abs(gl) + 1e-8), rtol=1e-9, atol=1e-18)
        p = new


def test_adam_two_steps_hand_computed():
    """Two Adam steps (b1 0.9, b2 0.999, eps 1e-8, lr 0.1) on one weight with
    gradients 1 then -2, worked by hand in exact rationals:
      step 1: mu = 0.1, nu = 0.001, m^ = 1, v^ = 1 -> p1 = p0 - 0.1 / (1 + 1e-8)
      step 2: mu = 0.9 * 0.1 - 0.2 = -0.11, nu = 0.999 * 0.001 + 0.001 * 4 = 0.004999,
              m^ = -0.11 / 0.19 = -11/19, v^ = 0.004999 / 0.001999 = 4999/1999,
              p2 = p1 + 0.1 * (11/19) / (sqrt(4999/1999) + 1e-8)
    and with the global-norm clip at 0.5 the same gradients enter as 0.5 and -0.5:
      step 2: mu = 0.045 - 0.05 = -0.005, nu = 0.999 * 0.00025 + 0.00025 = 0.00049975,
              m^ = -0.005 / 0.19 = -1/38, v^ = 0.00049975 / 0.001999 = 0.25
              (exactly 1999/7996), p2 = p1 + 0.1 * (1/38) / (0.5 + 1e-8)."""
    p0 = {"w": np.array([0.3])}
    opt = {"lr": 0.1, "max_grad_norm": None}
    p1, st, _ = ppo.optimizer_update({"w": np.array([1.0])}, ppo.optimizer_init(p0), p0, opt)
    np.testing.assert_allclose(p1["w"], 0.3 - 0.1 / (1 + 1e-8), rtol=1e-14)
    p2, st, _ = ppo.optimizer_update({"w": np.array([-2.0])}, st, p1, opt)
    np.testing.assert_allclose(st["mu"]["w"], -0.11, rtol=1e-13)
    np.testing.assert_allclose(st["nu"]["w"], 0.004999, rtol=1e-13)
    np.testing.assert_allclose(p2["w"], p1["w"] + 0.1 * (11 / 19) / (np.sqrt(4999 / 1999) + 1e-8), rtol=1e-14)
    # the same two gradients through clip_by_global_norm(0.5)
    opt = {"lr": 0.1, "max_grad_norm": 0.5}
    q1, st, n1 = ppo.optimizer_update({"w": np.array([1.0])}, ppo.optimizer_init(p0), p0, opt)
    q2, st, n2 = ppo.optimizer_update({"w": np.array([-2.0])}, st, q1, opt)
    assert (n1, n2) == (1.0, 2.0)
    np.testing.assert_allclose(st["mu"]["w"], -0.005, rtol=1e-13)
    np.testing.assert_allclose(st["nu"]["w"], 0.00049975, rtol=1e-13)
    np.testing.assert_allclose(q2["w"], q1["w"] + 0.1 * (1 / 38) / (0.5 + 1e-8), rtol=1e-14)
