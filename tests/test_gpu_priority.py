"""Parity of RecurrentPuPO's V-trace advantages
(boonta/algorithms/recurrent_pupo.py:210-220; ``ppo_vtrace_f32``) and its
prioritised env selection
(boonta/algorithms/recurrent_pupo.py:226-236; ``ppo_priority_choice_f32``)
against the oracle (oracle/priority.py) on the same seeded V-trace-shaped
advantages.

Tolerances (written here): probabilities 1e-5 relative (float32 priority
sums against the oracle's float64); indices bit-exact against the oracle's
draw on the kernel's own probabilities wherever the draw lies more than
1e-12 of the total from a cumulative boundary (at least 99.9 % of draws),
weights 2e-6 relative to (N p[idx]) ** -beta on those probabilities; against
the oracle's float64 probabilities, at least 95 % of indices equal and the
rest neighbours, weights 1e-4 relative where the indices agree.
"""
import numpy as np
import pytest
import torch

from boonta_amd import _lib
from boonta_amd.algorithms.pupo import prioritized_choice, vtrace
from oracle import gae as ogae
from boonta_amd.random import key as make_key
from oracle import priority

pytestmark = pytest.mark.gpu

CASES = [
    # (T, N, width, exponent, beta): the recurrent workload's 64 x 1024 envs
    # drawing 256-env minibatches; ragged, one-env, maximum and wide draws
    (64, 1024, 256, 0.6, 0.4),
    (7, 1000, 1000, 1.0, 1.0),
    (3, 1, 5, 0.6, 0.4),
    (2, 16384, 4096, 0.5, 0.7),
    (16, 3000, 20000, 0.8, 0.0),
]


@pytest.mark.parametrize("T,N,width,exponent,beta", CASES)
def test_priority_choice_matches_the_oracle(T, N, width, exponent, beta):
    rng = np.random.default_rng(T * 7919 + N)
    adv = (rng.standard_normal((T, N)) * rng.uniform(0.1, 3.0, N)).astype(np.float32)
    k = make_key(1000 + N)
    idx, w, prob = prioritized_choice(torch.from_numpy(adv).cuda(), k, width, exponent, beta)
    torch.cuda.synchronize()
    idx, w, prob = idx.cpu().numpy(), w.cpu().numpy(), prob.cpu().numpy()
    i_or, w_or, p_or, _ = priority.priority_choice(adv, k, width, exponent, beta)
    np.testing.assert_allclose(prob, p_or, rtol=1e-5, atol=1e-9)
    assert idx.min() >= 0 and idx.max() < N
    # the draw on the kernel's own float32 probabilities: exact but for draws
    # within float64 rounding of a boundary
    i_own, margin = priority.choice(k, prob.astype(np.float64), width)
    ok = margin > 1e-12
    assert ok.mean() >= 0.999
    np.testing.assert_array_equal(idx[ok], i_own[ok])
    np.testing.assert_allclose(w, (N * prob[idx].astype(np.float64)) ** -beta, rtol=2e-6)
    # against the oracle's float64 probabilities: neighbours at worst
    same = idx == i_or
    assert same.mean() >= 0.95
    assert np.abs(idx - i_or).max() <= 1
    np.testing.assert_allclose(w[same], w_or[same], rtol=1e-4)
    # against jax's float32 typing of the cumsum and r (sequential order):
    # at most 0.6 % of draws differ, each by one env
    i_f32 = priority.choice_f32(k, prob, width)
    assert (idx != i_f32).mean() <= 0.006
    assert np.abs(idx - i_f32).max() <= 1

def test_all_zero_advantages_draw_uniformly_and_a_device_key_matches_a_host_key():
    T, N, width = 4, 512, 2048
    adv = torch.zeros(T, N, device="cuda")
    k = make_key(3)
    idx, w, prob = prioritized_choice(adv, k, width, 0.6, 0.4)
    kd = torch.from_numpy(np.asarray(k, np.uint32).view(np.int32).copy()).cuda()
    idx2, w2, prob2 = prioritized_choice(adv, kd, width, 0.6, 0.4)
    torch.cuda.synchronize()
    assert torch.equal(idx, idx2) and torch.equal(w, w2)
    # (0 + 1e-6) / (0 + 1e-6) = 1 for every env: equal weights on a total of N
    np.testing.assert_allclose(prob.cpu().numpy(), 1.0, rtol=1e-6)
    i_or, _, _, margin = priority.priority_choice(np.zeros((T, N)), k, width, 0.6, 0.4)
    ok = margin > 1e-12
    np.testing.assert_array_equal(idx.cpu().numpy()[ok], i_or[ok])



@pytest.mark.parametrize("T,N,chunks", [(64, 1024, 0), (64, 1024, 1), (7, 100, 3), (1, 5, 0)])
def test_vtrace_matches_the_oracle_and_explicit_clipped_weights(T, N, chunks):
    """rho = min(ratio, advantage_clip), c = min(ratio, trace_clip) on the
    env-major ratio (recurrent_pupo.py:210-220): against the oracle's GAE
    with those weights (1e-5, the reference GAE test's tolerance), and
    bit-identical to ppo_gae_f32 given the same weights as arrays."""
    g = np.random.default_rng(T * 31 + N)
    r = g.normal(size=(T, N)).astype(np.float32)
    v = g.normal(size=(T, N)).astype(np.float32)
    b = g.normal(size=N).astype(np.float32)
    te = g.random((T, N)) < 0.02
    tr = (g.random((T, N)) < 0.01) & ~te
    ratio = g.uniform(0.3, 2.0, (N, T)).astype(np.float32)
    ratio[:, : max(T // 4, 1)] = 1.0    # the first minibatch's ratios are ones
    aclip, cclip = 1.0, 0.9
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    adv, ret = vtrace(d(r), d(te), d(tr), d(v), d(b), d(ratio), 0.99, 0.95, aclip, cclip, chunks)
    rho = np.minimum(ratio.T, np.float32(aclip))
    c = np.minimum(ratio.T, np.float32(cclip))
    exp_a, exp_r = ogae.gae(r, te, tr, v, b, 0.99, 0.95, rho=rho.astype(np.float64), c=c.astype(np.float64))
    np.testing.assert_allclose(adv.cpu().numpy(), exp_a, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(ret.cpu().numpy(), exp_r, rtol=1e-5, atol=1e-5)
    a2 = torch.empty(T, N, device="cuda")
    r2 = torch.empty(T, N, device="cuda")
    u8 = lambda x: d(x.astype(np.uint8))
    st = torch.cuda.current_stream().cuda_stream
    R, TE, TR, V, B, RHO, C = d(r), u8(te), u8(tr), d(v), d(b), d(rho), d(c)
    _lib.call("ppo_gae_f32", st, R.data_ptr(), TE.data_ptr(), TR.data_ptr(), V.data_ptr(), B.data_ptr(),
              RHO.data_ptr(), C.data_ptr(), a2.data_ptr(), r2.data_ptr(), T, N, 0.99, 0.95, chunks)
    torch.cuda.synchronize()
    assert torch.equal(adv, a2) and torch.equal(ret, r2)


def test_vtrace_propagates_a_nan_ratio():
    """jnp.minimum(NaN, clip) is NaN: a diverged ratio must show up as NaN
    advantages in its env column (at its step and every earlier one), not as
    a silently clipped weight; the other columns stay finite and exact."""
    T, N = 12, 70
    g = np.random.default_rng(5)
    r = g.normal(size=(T, N)).astype(np.float32)
    v = g.normal(size=(T, N)).astype(np.float32)
    b = g.normal(size=N).astype(np.float32)
    te = np.zeros((T, N), bool)
    tr = np.zeros((T, N), bool)
    ratio = g.uniform(0.3, 2.0, (N, T)).astype(np.float32)
    ratio[3, 7] = np.nan
    ratio[65, 0] = np.nan
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    adv, ret = vtrace(d(r), d(te), d(tr), d(v), d(b), d(ratio), 0.99, 0.95, 1.0, 0.9, 0)
    torch.cuda.synchronize()
    rho = np.minimum(ratio.T, np.float32(1.0)).astype(np.float64)
    c = np.minimum(ratio.T, np.float32(0.9)).astype(np.float64)
    exp_a, exp_r = ogae.gae(r, te, tr, v, b, 0.99, 0.95, rho=rho, c=c)
    got = adv.cpu().numpy()
    assert np.isnan(got[:8, 3]).all() and np.isfinite(got[8:, 3]).all()
    assert np.isnan(got[0, 65]) and np.isfinite(got[1:, 65]).all()
    assert np.isfinite(np.delete(got, [3, 65], axis=1)).all()
    np.testing.assert_allclose(got, exp_a, rtol=1e-5, atol=1e-5, equal_nan=True)
    np.testing.assert_allclose(ret.cpu().numpy(), exp_r, rtol=1e-5, atol=1e-5, equal_nan=True)
