"""Oracle networks (test infrastructure only): float64 forward and hand-written
backward for the torsos and heads on boonta's PPO learner path.

A network is described by a plain ``plan`` dict (stage lists with parameter
paths; see ``boonta_amd.networks.Network.plan``), so this module needs nothing
from the product.  Restated semantics:

- ``Network.__call__`` boonta/networks/network.py:18-49: feature extractor,
  optional recurrent torso, then the head; prev action/reward zeroed at done
  (:29-36; unused by the MLP configs).
- ``FeatureExtractor`` boonta/networks/feature_extractor.py:15-31 (observation
  extractor only).
- ``ActorCritic`` boonta/networks/actor_critic.py:11-14: actor distribution and
  ``critic(x).astype(float32)``.
- flax 0.12.8 ``Dense`` (y = x W + b, kernel [in, out]), ``LayerNorm``
  (epsilon 1e-6, fast variance E[x^2] - E[x]^2 clipped at 0, scale and bias),
  ``relu``/``tanh``/``silu``; ``GRUCell`` (gates r, z from input and recurrent
  projections, n = tanh(W_in x + b_in + r * (W_hn h + b_hn)),
  h' = (1 - z) n + z h).
- ``RNN`` + ``reset_carry`` boonta/networks/blocks/rnn.py:11-54: the carry is
  replaced by the zero initial carry wherever ``done[b, t]`` before the cell
  step at t.
- Distributions boonta/networks/distributions.py:8-57 over distrax 0.1.9:
  Categorical logits = log_softmax(preferences / temperature), Gaussian
  sigma = temperature * (softplus(scale) + 1e-3).
"""
from __future__ import annotations

import math

import numpy as np

# working precision: float64 for every check; bench.py's CPU baseline times
# the same code in float32 (oracle.working_precision)
FT = np.float64


def get(params, path):
    node = params
    for k in path:
        node = node[k]
    return node


def set_in(tree, path, value):
    node = tree
    for k in path[:-1]:
        node = node.setdefault(k, {})
    node[path[-1]] = value


def add_in(tree, path, value):
    node = tree
    for k in path[:-1]:
        node = node.setdefault(k, {})
    if path[-1] in node:
        node[path[-1]] = node[path[-1]] + value
    else:
        node[path[-1]] = value


# ----------------------------------------------------------------- activations
def act_fwd(fn, x):
    if fn == "relu":
        return np.maximum(x, 0.0)
    if fn == "tanh":
        return np.tanh(x)
    if fn == "silu":
        return x / (1.0 + np.exp(-x))
    raise ValueError(fn)


def act_bwd(fn, x, y, dy):
    if fn == "relu":
        # jax.nn.relu's derivative at 0 is 0
        return dy * (x > 0)
    if fn == "tanh":
        return dy * (1.0 - y * y)
    if fn == "silu":
        s = 1.0 / (1.0 + np.exp(-x))
        return dy * (s * (1.0 + x * (1.0 - s)))
    raise ValueError(fn)


# ----------------------------------------------------------------- bf16 casts
def bf16(x):
    """Round to the nearest-even bfloat16 value, via float32 (XLA rounds its
    fp32 results to bf16), returned in the working precision."""
    a = np.ascontiguousarray(np.asarray(x, FT).astype(np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return (u & 0xFFFFFFFF).astype(np.uint32).view(np.float32).astype(FT)


def _cast(x, dtype):
    return bf16(x) if dtype == "bfloat16" else x


# ---------------------------------------------------------------- stage lists
def stages_forward(params, stages, x, dtype="float32"):
    """Runs a stage list on x [rows, features]; returns (y, caches).

    With dtype "bfloat16" the flax mixed-precision casts are applied
    (boonta/networks/README.md:73-77): a Dense casts its input, kernel and bias
    to bf16, its dot returns bf16 (fp32 accumulation) and the bias add is a
    bf16 add; LayerNorm computes in fp32 and returns bf16; activations run on
    bf16 values."""
    caches = []
    for st in stages:
        op = st["op"]
        if op == "dense":
            p = get(params, st["path"])
            x = _cast(x, dtype)
            w = _cast(np.asarray(p["kernel"], FT), dtype)
            y = _cast(x @ w, dtype)
            if st.get("bias", True):
                y = _cast(y + _cast(np.asarray(p["bias"], FT), dtype), dtype)
            caches.append(x)
            x = y
        elif op == "layernorm":
            p = get(params, st["path"])
            mean = x.mean(-1, keepdims=True)
            var = np.maximum((x * x).mean(-1, keepdims=True) - mean * mean, 0.0)
            rstd = 1.0 / np.sqrt(var + st.get("eps", 1e-6))
            xhat = (x - mean) * rstd
            caches.append((xhat, rstd))
            x = _cast(xhat * np.asarray(p["scale"], FT) + np.asarray(p["bias"], FT), dtype)
        elif op == "act":
            y = act_fwd(st["fn"], x)
            if st["fn"] != "relu":
                y = _cast(y, dtype)
            caches.append((x, y))
            x = y
        else:
            raise ValueError(op)
    return x, caches


def stages_backward(params, stages, caches, dy, grads, need_dx=True, dtype="float32"):
    """Back-propagates dy through a stage list, adding parameter gradients
    into ``grads`` (same nesting as params).  Returns dx (or None).

    With dtype "bfloat16", every cotangent of a bf16 value is bf16 (the
    transposes of jax's casts): a Dense's input cotangent and its kernel and
    bias gradients are bf16 results converted to fp32, and LayerNorm's input
    cotangent is rounded to bf16."""
    dy = _cast(dy, dtype)
    for i in range(len(stages) - 1, -1, -1):
        st, cache = stages[i], caches[i]
        op = st["op"]
        if op == "dense":
            p = get(params, st["path"])
            x = cache
            add_in(grads, tuple(st["path"]) + ("kernel",), _cast(x.T @ dy, dtype))
            if st.get("bias", True):
                add_in(grads, tuple(st["path"]) + ("bias",), _cast(dy.sum(0), dtype))
            if i == 0 and not need_dx:
                return None
            dy = _cast(dy @ _cast(np.asarray(p["kernel"], FT), dtype).T, dtype)
        elif op == "layernorm":
            p = get(params, st["path"])
            xhat, rstd = cache
            add_in(grads, tuple(st["path"]) + ("scale",), (dy * xhat).sum(0))
            add_in(grads, tuple(st["path"]) + ("bias",), dy.sum(0))
            g = dy * np.asarray(p["scale"], FT)
            dy = _cast(rstd * (g - g.mean(-1, keepdims=True)
                               - xhat * (g * xhat).mean(-1, keepdims=True)), dtype)
        elif op == "act":
            x, y = cache
            dy = act_bwd(st["fn"], x, y, dy)
            if st["fn"] != "relu":
                dy = _cast(dy, dtype)
    return dy


# ------------------------------------------------------------------------ GRU
def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def gru_forward(params, torso, x, done, carry):
    """x [B, T, in], done [B, T] bool, carry [B, H] -> (outputs [B, T, H], final, cache).

    Before step t the carry is reset to zeros where done[:, t]
    (boonta/networks/blocks/rnn.py:42-45)."""
    p = get(params, torso["path"])
    k = lambda n: np.asarray(p[n]["kernel"], FT)
    b = lambda n: np.asarray(p[n]["bias"], FT)
    B, T, _ = x.shape
    H = torso["features"]
    xr = x @ k("ir") + b("ir")
    xz = x @ k("iz") + b("iz")
    xn = x @ k("in") + b("in")
    h = np.asarray(carry, FT)
    out = np.zeros((B, T, H), FT)
    cache = []
    for t in range(T):
        hp = np.where(done[:, t:t + 1], 0.0, h)
        r = _sig(xr[:, t] + hp @ k("hr"))
        z = _sig(xz[:, t] + hp @ k("hz"))
        hn = hp @ k("hn") + b("hn")
        n = np.tanh(xn[:, t] + r * hn)
        h = (1.0 - z) * n + z * hp
        out[:, t] = h
        cache.append((hp, r, z, hn, n))
    return out, h, (x, done, cache)


def gru_backward(params, torso, cache, dout, grads):
    """BPTT of gru_forward.  Returns dx [B, T, in]; the initial carry gets no
    gradient (it is data in RecurrentPPO.update)."""
    path = tuple(torso["path"])
    p = get(params, path)
    k = lambda n: np.asarray(p[n]["kernel"], FT)
    x, done, steps = cache
    B, T, _ = x.shape
    H = torso["features"]
    dh = np.zeros((B, H), FT)
    dxr = np.zeros((B, T, H), FT)
    dxz = np.zeros((B, T, H), FT)
    dxn = np.zeros((B, T, H), FT)
    dWhr = np.zeros((H, H), FT)
    dWhz = np.zeros((H, H), FT)
    dWhn = np.zeros((H, H), FT)
    dbhn = np.zeros(H, FT)
    for t in range(T - 1, -1, -1):
        hp, r, z, hn, n = steps[t]
        dh = dh + dout[:, t]
        dn = dh * (1.0 - z)
        dz = dh * (hp - n)
        dhp = dh * z
        dan = dn * (1.0 - n * n)           # pre-tanh
        dr = dan * hn
        dhn = dan * r
        daz = dz * z * (1.0 - z)
        dar = dr * r * (1.0 - r)
        dxr[:, t], dxz[:, t], dxn[:, t] = dar, daz, dan
        dWhr += hp.T @ dar
        dWhz += hp.T @ daz
        dWhn += hp.T @ dhn
        dbhn += dhn.sum(0)
        dhp = dhp + dar @ k("hr").T + daz @ k("hz").T + dhn @ k("hn").T
        dh = np.where(done[:, t:t + 1], 0.0, dhp)
    xf = x.reshape(B * T, -1)
    for name, d in (("ir", dxr), ("iz", dxz), ("in", dxn)):
        df = d.reshape(B * T, H)
        add_in(grads, path + (name, "kernel"), xf.T @ df)
        add_in(grads, path + (name, "bias"), df.sum(0))
    add_in(grads, path + ("hr", "kernel"), dWhr)
    add_in(grads, path + ("hz", "kernel"), dWhz)
    add_in(grads, path + ("hn", "kernel"), dWhn)
    add_in(grads, path + ("hn", "bias"), dbhn)
    dx = dxr @ k("ir").T + dxz @ k("iz").T + dxn @ k("in").T
    return dx


# -------------------------------------------------------------- distributions
LOG_2PI = math.log(2.0 * math.pi)


def softplus(x):
    return np.logaddexp(0.0, x)


def categorical_stats(logits, action):
    """log_prob(action) and entropy of distrax.Categorical(log_softmax(logits))
    (boonta/networks/distributions.py:8-19,32-38)."""
    z = logits - logits.max(-1, keepdims=True)
    logp = z - np.log(np.exp(z).sum(-1, keepdims=True))
    p = np.exp(logp)
    lp = np.take_along_axis(logp, action[:, None].astype(np.int64), -1)[:, 0]
    ent = -(p * logp).sum(-1)
    return lp, ent, (logp, p, ent)


def categorical_grad(cache, action, g_lp, g_ent):
    """d/dlogits of g_lp * log_prob + g_ent * entropy (row-wise weights)."""
    logp, p, ent = cache
    onehot = np.zeros_like(p)
    onehot[np.arange(len(action)), action.astype(np.int64)] = 1.0
    return g_lp[:, None] * (onehot - p) - g_ent[:, None] * p * (logp + ent[:, None])


def gaussian_sigma(raw_scale, temperature=1.0):
    return temperature * (softplus(raw_scale) + 1e-3)


def gaussian_stats(mean, sigma, action):
    """MultivariateNormalDiag log_prob/entropy (distributions.py:49-57)."""
    zs = (action - mean) / sigma
    lp = (-0.5 * zs * zs - np.log(sigma) - 0.5 * LOG_2PI).sum(-1)
    ent = np.broadcast_to((0.5 + 0.5 * LOG_2PI + np.log(sigma)), mean.shape).sum(-1)
    return lp, ent


def gaussian_grad(mean, sigma, action, g_lp, g_ent):
    """Returns (dmean [rows, D], dsigma [rows, D])."""
    d = action - mean
    dmean = g_lp[:, None] * d / (sigma * sigma)
    dsig = g_lp[:, None] * (d * d / sigma ** 3 - 1.0 / sigma) + g_ent[:, None] / sigma
    return dmean, dsig


# -------------------------------------------------------------- whole network
def forward(params, plan, obs):
    """MLP network forward on obs [rows, obs_dim].  Returns (head, value, cache),
    head being logits [rows, A] or mean [rows, D] (the heads' outputs are cast
    to fp32 before the distribution: distributions.py:35, actor_critic.py:14)."""
    dt = plan.get("compute_dtype", "float32")
    x = np.asarray(obs, FT)
    h, c_trunk = stages_forward(params, plan["trunk"], x, dt)
    head, c_actor = stages_forward(params, plan["actor"], h, dt)
    val, c_critic = stages_forward(params, plan["critic"], h, dt)
    return head, val[:, 0], (c_trunk, c_actor, c_critic)


def backward(params, plan, cache, dhead, dvalue, grads):
    dt = plan.get("compute_dtype", "float32")
    c_trunk, c_actor, c_critic = cache
    need = len(plan["trunk"]) > 0
    dh = stages_backward(params, plan["actor"], c_actor, dhead, grads, need_dx=need, dtype=dt)
    dh2 = stages_backward(params, plan["critic"], c_critic, dvalue[:, None], grads, need_dx=need, dtype=dt)
    if need:
        # two bf16 cotangents of the shared features add in bf16
        stages_backward(params, plan["trunk"], c_trunk, _cast(dh + dh2, dt), grads, need_dx=False, dtype=dt)


def recurrent_forward(params, plan, obs, done, carry):
    """Recurrent network on obs [B, T, obs_dim], done [B, T]; returns
    (head [B, T, ...], value [B, T], final carry, cache)."""
    B, T, D = obs.shape
    x = np.asarray(obs, FT).reshape(B * T, D)
    e, c_trunk = stages_forward(params, plan["trunk"], x)
    seq, final, c_gru = gru_forward(params, plan["torso"], e.reshape(B, T, -1), done, carry)
    h = seq.reshape(B * T, -1)
    head, c_actor = stages_forward(params, plan["actor"], h)
    val, c_critic = stages_forward(params, plan["critic"], h)
    return (head.reshape(B, T, -1), val[:, 0].reshape(B, T), final,
            (c_trunk, c_gru, c_actor, c_critic, (B, T)))


def recurrent_backward(params, plan, cache, dhead, dvalue, grads):
    c_trunk, c_gru, c_actor, c_critic, (B, T) = cache
    dh = stages_backward(params, plan["actor"], c_actor, dhead.reshape(B * T, -1), grads)
    dh = dh + stages_backward(params, plan["critic"], c_critic,
                              dvalue.reshape(B * T, 1), grads)
    de = gru_backward(params, plan["torso"], c_gru, dh.reshape(B, T, -1), grads)
    stages_backward(params, plan["trunk"], c_trunk, de.reshape(B * T, -1), grads,
                    need_dx=False)
