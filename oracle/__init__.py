"""CPU oracle for the PPO learner update — TEST INFRASTRUCTURE ONLY.

A float64 numpy (and plain C, for the integer PRNG work) restatement of
boonta's ``PPO.update`` / ``RecurrentPPO.update`` path, each function citing the
reference file:line it follows.  It is the checker for the HIP product path:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and never as the thing measured or shipped.

Parity status of each part (what pins it):

- ``prng``: Threefry-2x32-20 pinned by the Random123 known-answer vectors and
  by jax's documented ``split(key(0))`` value; the permutation composition is
  pinned by invariants and brute force (parity with a live jax: unpinned).
- ``gae``: pinned by the reference's own recursion test construction and by
  closed forms (no dones, lambda = 0, truncation).
- ``nets``: Dense / activations / LayerNorm / GRU backward pinned by float64
  finite differences; the GRU recurrence against torch.nn.GRUCell (float64,
  with resets) and the reference's torso invariants (reset forgets the past,
  stepped == chunked); the LayerNorm forward against
  torch.nn.functional.layer_norm; the bf16 casts against torch's CPU
  bfloat16.  Flax's exact op order: within tolerance only.
- ``ppo.loss_terms``: closed forms (ratio 1 at replay, clip fraction, KL 0) and
  finite differences of the scalar loss.
- ``sample``: the rollout-side Gumbel-max / Gaussian draws pinned by uniform
  endpoints on hand-computed words, chi-square of Gumbel-max frequencies,
  normal moments and a Kolmogorov-Smirnov test, and scipy's log-densities
  (parity with a live jax.random bit stream: unpinned).
- ``priority``: RecurrentPuPO's prioritised env selection, pinned by the
  closed form of equal priorities, a single-env distribution, a chi-square
  test of draw frequencies and the weights' closed form (parity with a live
  ``jax.random.choice`` stream: unpinned).
- ``ppo.optimizer_update``: closed forms of Adam: |update| = lr |g| /
  (|g| + eps) at every step of a constant gradient (bias corrections and
  moment decays at counts 1-5), a two-step case worked by hand in exact
  rationals with and without the global-norm clip, and clip invariants.

Everything runs in float64; ``working_precision(np.float32)`` switches the
network and update restatements to float32 for ``bench.py``'s CPU baseline
(a timing, never a check).
"""
from __future__ import annotations

import contextlib


@contextlib.contextmanager
def working_precision(dtype):
    """Runs ``nets`` and ``ppo`` in ``dtype`` inside the block."""
    from . import nets, ppo
    old = nets.FT, ppo.FT
    nets.FT = ppo.FT = dtype
    try:
        yield
    finally:
        nets.FT, ppo.FT = old
