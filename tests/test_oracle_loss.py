"""The oracle's PPO loss where its clips bind, and its explained variance,
against values worked by hand (boonta/algorithms/ppo.py:90-121 for the
clipped surrogate and the clipped value loss, :167-169 for the explained
variance; recurrent_ppo.py's loss is the same formula).

Every case states its arithmetic.  Mutated copies of the oracle's
``loss_terms`` (``max`` for ``min`` in the surrogate, the value clip taken
around the return or dropped, the mean of squared residuals or the sample
variance for the population variance, the entropy bonus's sign) must each
fail the closed form named beside it: the cases pin those terms, not just the
oracle's agreement with itself."""
import inspect
import textwrap

import numpy as np
import pytest

from oracle import ppo

EPS = 0.2
CFG = {"clip_coefficient": EPS, "clip_value_loss": True, "entropy_coefficient": 0.01, "value_coefficient": 0.5}


def one_row(loss_terms, ratio, adv, value=0.0, old_value=0.0, ret=0.0, clip_value=True, ent=0.0):
    """loss_terms on a single row whose new/old log-prob difference is log(ratio)."""
    old = np.array([-1.0])
    logp = old + np.log(ratio)
    cfg = dict(CFG, clip_value_loss=clip_value)
    return loss_terms(logp, np.array([ent]), np.array([value]), old, np.array([old_value]), np.array([adv]),
                      np.array([ret]), cfg)


# (ratio, advantage, actor loss, d loss / d logp); eps = 0.2, one row
#   r = 1.5 > 1.2, A =  2: min(3.0, 1.2 * 2 = 2.4)  = 2.4  -> loss -2.4, clipped branch, flat: grad 0
#   r = 1.5 > 1.2, A = -2: min(-3.0, -2.4)          = -3.0 -> loss  3.0, grad -A r = 3.0
#   r = 0.5 < 0.8, A =  2: min(1.0, 0.8 * 2 = 1.6)  = 1.0  -> loss -1.0, grad -A r = -1.0
#   r = 0.5 < 0.8, A = -2: min(-1.0, -1.6)          = -1.6 -> loss  1.6, clipped branch, flat: grad 0
#   r = 1.1 inside,  A = 2: min(2.2, 2.2) (tie)     = 2.2  -> loss -2.2, grad -A r = -2.2 (both branches
#                                                             carry the same slope inside the clip range)
SURROGATE = [(1.5, 2.0, -2.4, 0.0), (1.5, -2.0, 3.0, 3.0), (0.5, 2.0, -1.0, -1.0), (0.5, -2.0, 1.6, 0.0),
             (1.1, 2.0, -2.2, -2.2)]

# (v, v_old, R, clip_value_loss, critic loss, d critic / d v); eps = 0.2
#   v - v_old =  0.5 > eps, R = 0: 0.5 (1.5)^2 = 1.125 vs clipped 0.5 (1.2)^2 = 0.72  -> 1.125, grad v - R = 1.5
#   v - v_old =  0.5 > eps, R = 3: 0.5 (-1.5)^2 = 1.125 vs 0.5 (1.2 - 3)^2 = 1.62     -> 1.62, clipped: grad 0
#   v - v_old = -0.5 < -eps, R = 2: 0.5 (-1.5)^2 = 1.125 vs 0.5 (0.8 - 2)^2 = 0.72    -> 1.125, grad -1.5
#   v - v_old = -0.5 < -eps, R = -1: 1.125 vs 0.5 (0.8 + 1)^2 = 1.62                  -> 1.62, grad 0
#   the last two again without the value clip: 0.5 (v - R)^2 = 1.125 and 1.125, grads -1.5 and 1.5
VALUE = [(1.5, 1.0, 0.0, True, 1.125, 1.5), (1.5, 1.0, 3.0, True, 1.62, 0.0), (0.5, 1.0, 2.0, True, 1.125, -1.5),
         (0.5, 1.0, -1.0, True, 1.62, 0.0), (0.5, 1.0, 2.0, False, 1.125, -1.5), (0.5, 1.0, -1.0, False, 1.125, 1.5)]


def check_surrogate(loss_terms):
    for ratio, adv, want, dwant in SURROGATE:
        loss, logs, (g_logp, _, _) = one_row(loss_terms, ratio, adv)
        np.testing.assert_allclose(logs["actor/loss"], want, rtol=1e-12, err_msg=f"r={ratio} A={adv}")
        np.testing.assert_allclose(g_logp[0], dwant, rtol=1e-12, atol=1e-15, err_msg=f"r={ratio} A={adv}")
        assert logs["actor/clip_fraction"] == (1.0 if abs(ratio - 1.0) > EPS else 0.0)
        np.testing.assert_allclose(logs["actor/approximate_kl"], -np.log(ratio), rtol=1e-12)


def check_value(loss_terms):
    for v, vo, ret, clip, want, dwant in VALUE:
        loss, logs, (_, _, g_value) = one_row(loss_terms, 1.0, 0.0, value=v, old_value=vo, ret=ret,
                                              clip_value=clip)
        np.testing.assert_allclose(logs["critic/loss"], want, rtol=1e-12, err_msg=f"v={v} vo={vo} R={ret}")
        # the loss carries the critic term at value_coefficient; g_value is d loss / d v
        np.testing.assert_allclose(g_value[0], 0.5 * dwant, rtol=1e-12, atol=1e-15)


def check_total(loss_terms):
    # loss = actor - c_e * entropy + c_v * critic, on two rows:
    #   row 0: r = 1.5, A = 2 -> pg term 2.4; v 1.5, v_old 1.0, R 0 -> 1.125; entropy 0.7
    #   row 1: r = 0.5, A = 2 -> pg term 1.0; v 0.5, v_old 1.0, R -1 -> 1.62; entropy 1.1
    #   actor = -(2.4 + 1.0) / 2 = -1.7; critic = (1.125 + 1.62) / 2 = 1.3725; entropy = 0.9
    #   loss = -1.7 - 0.01 * 0.9 + 0.5 * 1.3725 = -1.02275
    old = np.array([-1.0, -2.0])
    logp = old + np.log([1.5, 0.5])
    loss, logs, (_, g_ent, _) = loss_terms(logp, np.array([0.7, 1.1]), np.array([1.5, 0.5]), old,
                                           np.array([1.0, 1.0]), np.array([2.0, 2.0]), np.array([0.0, -1.0]), CFG)
    np.testing.assert_allclose(logs["actor/loss"], -1.7, rtol=1e-12)
    np.testing.assert_allclose(logs["critic/loss"], 1.3725, rtol=1e-12)
    np.testing.assert_allclose(logs["actor/entropy"], 0.9, rtol=1e-12)
    np.testing.assert_allclose(loss, -1.02275, rtol=1e-12)
    np.testing.assert_allclose(g_ent, [-0.005, -0.005], rtol=1e-12)


def explained_variance(loss_terms, value, ret):
    n = len(value)
    _, logs, _ = loss_terms(np.zeros(n), np.zeros(n), np.asarray(value, float), np.zeros(n), np.asarray(value, float),
                            np.zeros(n), np.asarray(ret, float), CFG)
    return logs["critic/explained_variance"]


def check_explained_variance(loss_terms):
    rng = np.random.default_rng(3)
    R = rng.normal(size=64)
    # v = R + c: the residual is constant, its variance 0 -> exactly 1
    assert explained_variance(loss_terms, R + 0.75, R) == 1.0
    # a constant v: var(R - v) = var(R) -> 1 - var / (var + 1e-8), about 0
    np.testing.assert_allclose(explained_variance(loss_terms, np.full(64, 0.3), R),
                               1.0 - R.var() / (R.var() + 1e-8), rtol=0, atol=1e-15)
    # R = [0, 4], v = [0, 2]: R - v = [0, 2], population variances 1 and 4 -> 1 - 1 / (4 + 1e-8)
    np.testing.assert_allclose(explained_variance(loss_terms, [0.0, 2.0], [0.0, 4.0]), 1.0 - 1.0 / (4.0 + 1e-8),
                               rtol=1e-14)
    # a return variance the size of the 1e-8 guard tells population from sample variance:
    # R = [0, 2e-4], v = 0: var(R) = 1e-8 -> 1 - 1e-8 / 2e-8 = 0.5 (sample variances would give 1/3)
    np.testing.assert_allclose(explained_variance(loss_terms, [0.0, 0.0], [0.0, 2e-4]), 0.5, rtol=1e-9)


CHECKS = [check_surrogate, check_value, check_total, check_explained_variance]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_loss_closed_forms(check):
    check(ppo.loss_terms)


def mutated(old: str, new: str):
    """ppo.loss_terms with one source fragment replaced (a planted mistake)."""
    src = textwrap.dedent(inspect.getsource(ppo.loss_terms))
    assert src.count(old) == 1, old
    ns = dict(vars(ppo))
    exec(compile(src.replace(old, new), "<mutant>", "exec"), ns)
    return ns["loss_terms"]


MUTANTS = {  # name: (fragment, replacement, the closed form that must catch it)
    "max for min in the surrogate": ("actor = -np.minimum(pg1, pg2).mean()", "actor = -np.maximum(pg1, pg2).mean()",
                                     check_surrogate),
    "value clip around the return": ("vc = old_value + dv_clip", "vc = ret + _clip_and_grad(value - ret, -eps, eps)[0]",
                                     check_value),
    "mean square for the variance": ("1.0 - resid.var() / (ret.var() + 1e-8)",
                                     "1.0 - (resid ** 2).mean() / (ret.var() + 1e-8)", check_explained_variance),
    "sample variance": ("1.0 - resid.var() / (ret.var() + 1e-8)",
                        "1.0 - resid.var(ddof=1) / (ret.var(ddof=1) + 1e-8)", check_explained_variance),
    "no value clip": ("crit_rows = np.maximum(vl1, vl2)", "crit_rows = vl1", check_value),
    "entropy sign": ("loss = actor - cfg[\"entropy_coefficient\"] * entropy",
                     "loss = actor + cfg[\"entropy_coefficient\"] * entropy", check_total),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_every_planted_mistake_fails_its_closed_form(name):
    old, new, check = MUTANTS[name]
    bad = mutated(old, new)
    with np.errstate(all="ignore"), pytest.raises(AssertionError):
        check(bad)
