"""Pins the oracle's bf16 emulation (flax Dense / LayerNorm with
dtype=bfloat16, boonta/networks/README.md:73-77) against torch's CPU bfloat16,
an independent implementation of the same rounding and of a bf16 matmul with
fp32 accumulation (no GPU)."""
import numpy as np
import torch

from oracle import nets


def torch_bf16(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).to(torch.float32).numpy().astype(np.float64)


def test_rounding_matches_torch_bfloat16():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000) * 10.0 ** rng.integers(-6, 6, 10000),
                        # exact ties between two bf16 values: round half to even
                        1.0 + np.array([1, 3, 5, 7]) * 2.0 ** -8, -(1.0 + np.array([1, 3]) * 2.0 ** -8),
                        [0.0, -0.0, 1e-40, 3.0e38, np.inf, -np.inf]])
    np.testing.assert_array_equal(nets.bf16(x), torch_bf16(x))
    assert nets.bf16(1.0 + 2.0 ** -8) == 1.0            # tie to even (down)
    assert nets.bf16(1.0 + 3 * 2.0 ** -8) == 1.0 + 2.0 ** -6   # tie to even (up)


def test_bf16_dense_matches_a_bf16_matmul_with_fp32_accumulation():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 300))
    w = rng.standard_normal((300, 40)) / np.sqrt(300)
    b = 0.1 * rng.standard_normal(40)
    params = {"d": {"kernel": w, "bias": b}}
    y, _ = nets.stages_forward(params, [{"op": "dense", "path": ("d",), "in": 300, "out": 40}], x, "bfloat16")
    tx = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    tw = torch.from_numpy(w.astype(np.float32)).to(torch.bfloat16)
    tb = torch.from_numpy(b.astype(np.float32)).to(torch.bfloat16)
    ref = ((tx @ tw) + tb).to(torch.float32).numpy().astype(np.float64)
    # the two sums may round differently only where fp32 accumulation order flips a bf16 tie
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(y - ref) <= ulp)
    assert np.mean(y == ref) > 0.98


def test_bf16_layernorm_relu_rounds_once_after_the_normalisation():
    rng = np.random.default_rng(2)
    x = nets.bf16(rng.standard_normal((16, 512)))
    params = {"ln": {"scale": 1.0 + 0.1 * rng.standard_normal(512), "bias": 0.1 * rng.standard_normal(512)}}
    stages = [{"op": "layernorm", "path": ("ln",), "eps": 1e-6}, {"op": "act", "fn": "relu"}]
    y, _ = nets.stages_forward(params, stages, x, "bfloat16")
    # float64 LayerNorm from torch, rounded once to bf16, then ReLU
    ln = torch.nn.functional.layer_norm(torch.from_numpy(x), (512,), torch.from_numpy(params["ln"]["scale"]),
                                        torch.from_numpy(params["ln"]["bias"]), eps=1e-6).numpy()
    np.testing.assert_array_equal(y, np.maximum(torch_bf16(ln), 0.0))


def test_bf16_backward_rounds_every_cotangent():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((32, 24))
    params = {"d": {"kernel": rng.standard_normal((24, 8)), "bias": np.zeros(8)}}
    stages = [{"op": "dense", "path": ("d",), "in": 24, "out": 8}]
    _, caches = nets.stages_forward(params, stages, x, "bfloat16")
    grads = {}
    dy = rng.standard_normal((32, 8))
    dx = nets.stages_backward(params, stages, caches, dy, grads, dtype="bfloat16")
    for v in (dx, grads["d"]["kernel"], grads["d"]["bias"]):
        np.testing.assert_array_equal(v, nets.bf16(v))
    # and they are the bf16 roundings of the exact products of the bf16 operands
    xb, dyb, wb = nets.bf16(x), nets.bf16(dy), nets.bf16(params["d"]["kernel"])
    np.testing.assert_array_equal(grads["d"]["kernel"], nets.bf16(xb.T @ dyb))
    np.testing.assert_array_equal(dx, nets.bf16(dyb @ wb.T))
