"""Network descriptions for the learner, mirroring the flax compositions boonta's
PPO recipes build (``Network(feature_extractor=FeatureExtractor(...), torso=...,
head=ActorCritic(actor=Categorical|Gaussian(...), critic=...))``).

These classes carry structure only.  ``Network.plan(obs_dim)`` lowers a
composition into a plain stage plan the learner compiles into kernel launches,
and ``Network.init(key, obs_dim)`` draws parameters into a nested dict whose
nesting follows flax's naming (``layers_<i>`` inside ``Sequential``, a head's
layer sharing its scope, ``kernel``/``bias``/``scale``), so a parameter tree
keeps the shape of the reference's ``params["params"]``.

Reference modules mirrored:
  boonta/networks/network.py:13-55           Network
  boonta/networks/feature_extractor.py:10-31 FeatureExtractor
  boonta/networks/actor_critic.py:7-14       ActorCritic
  boonta/networks/heads.py:9-45              Categorical, Gaussian
  boonta/networks/blocks/rnn.py:30-59        RNN (+ flax GRUCell)
  boonta/networks/layers/identity.py         Identity
  hangar/recipes/recurrent_ppo_classic_control.py:19-28  SpreadScale
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field
from typing import Any, Callable

import numpy as np


# ----------------------------------------------------------------- initialisers
@dataclass(frozen=True)
class Initializer:
    kind: str
    scale: float = 1.0

    def __call__(self, rng: np.random.Generator, shape) -> np.ndarray:
        shape = tuple(shape)
        if self.kind == "zeros":
            return np.zeros(shape, np.float32)
        if self.kind == "constant":
            return np.full(shape, self.scale, np.float32)
        if self.kind == "lecun_normal":
            # variance_scaling(1, fan_in, truncated_normal): std / .8796 on [-2, 2]
            fan_in = shape[0] if len(shape) > 1 else 1
            std = np.sqrt(self.scale / fan_in) / 0.87962566103423978
            x = rng.standard_normal(shape)
            bad = np.abs(x) > 2
            while bad.any():
                x[bad] = rng.standard_normal(int(bad.sum()))
                bad = np.abs(x) > 2
            return (x * std).astype(np.float32)
        if self.kind == "orthogonal":
            rows, cols = shape[0], int(np.prod(shape[1:]))
            a = rng.standard_normal((max(rows, cols), min(rows, cols)))
            q, r = np.linalg.qr(a)
            q = q * np.sign(np.diag(r))
            if rows < cols:
                q = q.T
            return (self.scale * q[:rows, :cols]).reshape(shape).astype(np.float32)
        raise ValueError(self.kind)


def lecun_normal() -> Initializer:
    return Initializer("lecun_normal")


def orthogonal(scale: float = 1.0) -> Initializer:
    return Initializer("orthogonal", float(scale))


def zeros_init() -> Initializer:
    return Initializer("zeros")


def constant(value: float) -> Initializer:
    return Initializer("constant", float(value))


# ---------------------------------------------------------------------- modules
class Module:
    pass


@dataclass(frozen=True)
class Activation(Module):
    name: str

    def __call__(self, x):  # pragma: no cover - structure only
        raise TypeError("activations are compiled into kernels, not called")


relu = Activation("relu")
tanh = Activation("tanh")
silu = Activation("silu")
swish = silu


@dataclass(frozen=True)
class Dense(Module):
    features: int
    use_bias: bool = True
    kernel_init: Initializer = dataclasses.field(default_factory=lecun_normal)
    bias_init: Initializer = dataclasses.field(default_factory=zeros_init)
    dtype: Any = None


@dataclass(frozen=True)
class LayerNorm(Module):
    epsilon: float = 1e-6
    dtype: Any = None


@dataclass(frozen=True)
class Sequential(Module):
    layers: tuple

    def __init__(self, layers):
        object.__setattr__(self, "layers", tuple(layers))


@dataclass(frozen=True)
class Identity(Module):
    pass


@dataclass(frozen=True)
class FeatureExtractor(Module):
    observation_extractor: Module
    action_extractor: Module | None = None
    reward_extractor: Module | None = None
    done_extractor: Module | None = None


@dataclass(frozen=True)
class Categorical(Module):
    layer: Module
    reinterpreted_batch_ndims: int = 0


@dataclass(frozen=True)
class Gaussian(Module):
    layer: Module


@dataclass(frozen=True)
class SpreadScale(Module):
    """Mean from a Dense(action_dim, orthogonal(0.01)) and one state-independent
    raw scale per dimension, initialised to log(expm1(1 - 1e-3)) so that
    sigma = softplus(scale) + 1e-3 = 1 (recurrent_ppo_classic_control.py:19-28)."""
    action_dim: int
    kernel_init: Initializer = dataclasses.field(default_factory=lambda: orthogonal(0.01))
    scale_init: float = float(np.log(np.expm1(1.0 - 1e-3)))


@dataclass(frozen=True)
class ActorCritic(Module):
    actor: Module
    critic: Module


@dataclass(frozen=True)
class GRUCell(Module):
    features: int
    kernel_init: Initializer = dataclasses.field(default_factory=lecun_normal)
    recurrent_kernel_init: Initializer = dataclasses.field(default_factory=orthogonal)


@dataclass(frozen=True)
class RNN(Module):
    cell: GRUCell


@dataclass(frozen=True)
class Network(Module):
    feature_extractor: Module = Identity()
    torso: Module | None = None
    head: Module = Identity()

    # -------------------------------------------------------------- lowering
    def plan(self, obs_dim: int) -> dict:
        """Lowers the composition into the learner's stage plan (plain data)."""
        width = [obs_dim]
        dtypes = set()

        def lower(mod, path):
            stages = []
            if isinstance(mod, Identity) or mod is None:
                return stages
            if isinstance(mod, FeatureExtractor):
                if mod.action_extractor or mod.reward_extractor or mod.done_extractor:
                    raise NotImplementedError("only observation extractors are compiled")
                return lower(mod.observation_extractor, path + ("observation_extractor",))
            if isinstance(mod, Sequential):
                for i, layer in enumerate(mod.layers):
                    stages += lower(layer, path + (f"layers_{i}",))
                return stages
            if isinstance(mod, Dense):
                dtypes.add(_dtype_name(mod.dtype))
                st = {"op": "dense", "path": path, "in": width[0], "out": mod.features,
                      "bias": mod.use_bias}
                width[0] = mod.features
                return [st]
            if isinstance(mod, LayerNorm):
                dtypes.add(_dtype_name(mod.dtype))
                return [{"op": "layernorm", "path": path, "width": width[0], "eps": mod.epsilon}]
            if isinstance(mod, Activation):
                # Activations are not flax modules: they do not take a slot name.
                return [{"op": "act", "fn": mod.name}]
            if isinstance(mod, SpreadScale):
                st = {"op": "dense", "path": path + ("Dense_0",), "in": width[0],
                      "out": mod.action_dim, "bias": True, "spread_scale": path + ("scale",)}
                width[0] = mod.action_dim
                return [st]
            raise NotImplementedError(f"module {type(mod).__name__} is not compiled by the learner")

        trunk = lower(self.feature_extractor, ("feature_extractor",))
        trunk_width = width[0]
        torso = None
        if self.torso is not None:
            if not isinstance(self.torso, RNN) or not isinstance(self.torso.cell, GRUCell):
                raise NotImplementedError("the recurrent torso must be RNN(GRUCell)")
            torso = {"op": "gru", "path": ("torso", "cell"), "in": trunk_width,
                     "features": self.torso.cell.features}
            trunk_width = self.torso.cell.features
        if not isinstance(self.head, ActorCritic):
            raise NotImplementedError("the head must be an ActorCritic")
        actor_mod = self.head.actor
        width[0] = trunk_width
        if isinstance(actor_mod, Categorical):
            actor = lower(actor_mod.layer, ("head", "actor"))
            dist = {"kind": "categorical", "num": width[0]}
        elif isinstance(actor_mod, Gaussian):
            actor = lower(actor_mod.layer, ("head", "actor"))
            last = actor[-1]
            if last.get("spread_scale") is not None:
                dist = {"kind": "gaussian", "dim": width[0], "scale": last["spread_scale"]}
            else:
                if width[0] % 2:
                    raise ValueError("a Gaussian head's layer must output 2 * action_dim")
                dist = {"kind": "gaussian", "dim": width[0] // 2, "scale": None}
        else:
            raise NotImplementedError("the actor must be Categorical or Gaussian")
        width[0] = trunk_width
        critic = lower(self.head.critic, ("head", "critic"))
        if not critic or critic[-1]["op"] != "dense" or critic[-1]["out"] != 1:
            raise ValueError("the critic must end in Dense(1)")
        if not actor or actor[-1]["op"] != "dense":
            raise ValueError("the actor must end in a Dense layer")
        dtypes.discard(None)
        if len(dtypes) > 1:
            raise NotImplementedError("mixed compute dtypes are not compiled")
        return {
            "obs_dim": obs_dim,
            "compute_dtype": dtypes.pop() if dtypes else "float32",
            "trunk": trunk,
            "torso": torso,
            "actor": actor,
            "critic": critic,
            "dist": dist,
        }

    # ---------------------------------------------------------------- params
    def init(self, key, obs_dim: int) -> dict:
        """Parameters {"params": {...}} for this composition.  ``key`` is an
        int seed or uint32[2] key data; draws use numpy, so values differ from
        flax's initialisers bit for bit but follow the same distributions."""
        seed = int(np.asarray(key, dtype=np.uint64).ravel().sum()) if not isinstance(key, int) else key
        rng = np.random.default_rng(seed)
        plan = self.plan(obs_dim)
        params: dict = {}
        mods = _modules_by_path(self)

        def put(path, value):
            node = params
            for k in path[:-1]:
                node = node.setdefault(k, {})
            node[path[-1]] = value

        for st in plan["trunk"] + plan["actor"] + plan["critic"]:
            if st["op"] == "dense":
                mod = mods.get(tuple(st["path"]))
                kinit = mod.kernel_init if mod is not None else lecun_normal()
                binit = getattr(mod, "bias_init", zeros_init()) if mod is not None else zeros_init()
                put(tuple(st["path"]) + ("kernel",), kinit(rng, (st["in"], st["out"])))
                if st.get("bias", True):
                    put(tuple(st["path"]) + ("bias",), binit(rng, (st["out"],)))
                if st.get("spread_scale") is not None:
                    sp = mods[tuple(st["spread_scale"][:-1])]
                    put(tuple(st["spread_scale"]), np.full((st["out"],), sp.scale_init, np.float32))
            elif st["op"] == "layernorm":
                put(tuple(st["path"]) + ("scale",), np.ones(st["width"], np.float32))
                put(tuple(st["path"]) + ("bias",), np.zeros(st["width"], np.float32))
        if plan["torso"] is not None:
            cell = self.torso.cell
            H, I = plan["torso"]["features"], plan["torso"]["in"]
            base = tuple(plan["torso"]["path"])
            for g in ("ir", "iz", "in"):
                put(base + (g, "kernel"), cell.kernel_init(rng, (I, H)))
                put(base + (g, "bias"), np.zeros(H, np.float32))
            for g in ("hr", "hz", "hn"):
                put(base + (g, "kernel"), cell.recurrent_kernel_init(rng, (H, H)))
            put(base + ("hn", "bias"), np.zeros(H, np.float32))
        return {"params": params}


def _dtype_name(dtype) -> str | None:
    if dtype is None:
        return None
    name = getattr(dtype, "__name__", None) or str(dtype)
    name = name.replace("torch.", "").replace("jnp.", "")
    if name in ("bfloat16", "bf16"):
        return "bfloat16"
    if name in ("float32", "fp32", "f32"):
        return "float32"
    raise NotImplementedError(f"compute dtype {dtype!r}")


def _modules_by_path(net: Network) -> dict:
    out = {}

    def walk(mod, path):
        if isinstance(mod, FeatureExtractor):
            walk(mod.observation_extractor, path + ("observation_extractor",))
        elif isinstance(mod, Sequential):
            for i, layer in enumerate(mod.layers):
                walk(layer, path + (f"layers_{i}",))
        elif isinstance(mod, (Categorical, Gaussian)):
            walk(mod.layer, path)
        elif isinstance(mod, SpreadScale):
            out[path] = mod
            out[path + ("Dense_0",)] = Dense(mod.action_dim, kernel_init=mod.kernel_init)
        elif isinstance(mod, ActorCritic):
            walk(mod.actor, path + ("actor",))
            walk(mod.critic, path + ("critic",))
        elif isinstance(mod, (Dense, LayerNorm)):
            out[path] = mod

    walk(net.feature_extractor, ("feature_extractor",))
    walk(net.head, ("head",))
    return out
