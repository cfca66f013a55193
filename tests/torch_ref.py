"""Forward pass of a network plan in plain PyTorch fp32, used only to fill a
synthetic rollout's actions, log-probs and values on the device (the harness
side of a benchmark: it is never part of the learner update)."""
from __future__ import annotations

import torch


def _get(tree, path):
    for k in path:
        tree = tree[k]
    return tree


def _stages(params, stages, x):
    for st in stages:
        if st["op"] == "dense":
            p = _get(params, st["path"])
            x = x @ p["kernel"]
            if st.get("bias", True):
                x = x + p["bias"]
        elif st["op"] == "layernorm":
            p = _get(params, st["path"])
            x = torch.nn.functional.layer_norm(x, (x.shape[-1],), p["scale"], p["bias"], st.get("eps", 1e-6))
        elif st["op"] == "act":
            x = {"relu": torch.relu, "tanh": torch.tanh, "silu": torch.nn.functional.silu}[st["fn"]](x)
    return x


@torch.no_grad()
def forward(params, plan, obs: torch.Tensor):
    h = _stages(params, plan["trunk"], obs)
    return _stages(params, plan["actor"], h), _stages(params, plan["critic"], h)[..., 0]


@torch.no_grad()
def sample(params, plan, obs: torch.Tensor, generator: torch.Generator):
    """(action, log_prob, value) of the policy on obs [rows, obs_dim]."""
    head, value = forward(params, plan, obs)
    d = plan["dist"]
    if d["kind"] == "categorical":
        u = torch.rand(head.shape, device=head.device, generator=generator).clamp_min(1e-20)
        action = torch.argmax(head - torch.log(-torch.log(u)), dim=-1)
        logp = torch.log_softmax(head, -1).gather(-1, action[:, None])[:, 0]
        return action.to(torch.int32), logp, value
    D = d["dim"]
    if d.get("scale") is not None:
        raw = _get(params, d["scale"]).expand_as(head)
        mean = head
    else:
        mean, raw = head[:, :D], head[:, D:]
    sig = torch.nn.functional.softplus(raw) + 1e-3
    a = mean + sig * torch.randn(mean.shape, device=head.device, generator=generator)
    z = (a - mean) / sig
    logp = (-0.5 * z * z - torch.log(sig) - 0.5 * 1.8378770664093453).sum(-1)
    return a, logp, value


@torch.no_grad()
def recurrent_sample(params, plan, obs: torch.Tensor, first_done: torch.Tensor, carry0: torch.Tensor,
                     generator: torch.Generator):
    """Rollout-side pass of a recurrent plan over obs [T, N, obs_dim] from
    carry0 [N, H], resetting the carry where first_done [T, N]: returns
    (action [T, N], log_prob, value, carry [T, N, H]) with carry[t] the carry
    entering step t, as Anakin.rollout records it."""
    T, N, D = obs.shape
    t = plan["torso"]
    c = _get(params, t["path"])
    x = _stages(params, plan["trunk"], obs.reshape(T * N, D)).reshape(T, N, -1)
    xr = x @ c["ir"]["kernel"] + c["ir"]["bias"]
    xz = x @ c["iz"]["kernel"] + c["iz"]["bias"]
    xn = x @ c["in"]["kernel"] + c["in"]["bias"]
    h = carry0
    carries, outs = [], []
    for s in range(T):
        carries.append(h)
        hp = torch.where(first_done[s, :, None], torch.zeros_like(h), h)
        r = torch.sigmoid(xr[s] + hp @ c["hr"]["kernel"])
        z = torch.sigmoid(xz[s] + hp @ c["hz"]["kernel"])
        n = torch.tanh(xn[s] + r * (hp @ c["hn"]["kernel"] + c["hn"]["bias"]))
        h = (1.0 - z) * n + z * hp
        outs.append(h)
    feats = torch.stack(outs).reshape(T * N, -1)
    head = _stages(params, plan["actor"], feats)
    value = _stages(params, plan["critic"], feats)[..., 0]
    u = torch.rand(head.shape, device=head.device, generator=generator).clamp_min(1e-20)
    action = torch.argmax(head - torch.log(-torch.log(u)), dim=-1)
    logp = torch.log_softmax(head, -1).gather(-1, action[:, None])[:, 0]
    return (action.to(torch.int32).reshape(T, N), logp.reshape(T, N), value.reshape(T, N),
            torch.stack(carries))
