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
  finite differences; GRU forward by the reference's torso invariants
  (reset forgets the past, stepped == chunked).  Flax op order: unpinned
  (within tolerance only).
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
- ``ppo.optimizer_update``: closed form of Adam's first step
  (|update| = lr for |g| >> eps) and clip invariants; optax itself: unpinned.
"""
