// One categorical draw per row by a 16-lane group, shared by the sampling
// launch of the rollout step and the fused MLP step kernel: lane j0 of the
// group owns logits j0, j0 + 16, ... (A <= 128).  Follows
// boonta/networks/distributions.py:8-23 with distrax's normalisation and
// jax.random.gumbel (low-dynamic-range mode) on the key's Threefry stream:
//   logits = log_softmax(pref / T) (T <= 0: 0 at the greedy index, -inf
//   elsewhere); action = argmax(logits + gumbel) over the flat indices
//   row * A + j of the draw; log_prob = logits[action].
#pragma once
#include "common.h"
#include "threefry.h"

#include <math.h>

namespace ppo {
namespace cat {

constexpr int GROUP = 16;
constexpr int MAX_K = 8;  // logits per lane: A <= 128

__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = GROUP / 2; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, GROUP));
  return v;
}

__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = GROUP / 2; o; o >>= 1) v += __shfl_xor(v, o, GROUP);
  return v;
}

// (value, index) argmax across the group: larger value wins, the smaller
// index on equal values; `extra` travels with the winner.
__device__ __forceinline__ void group_argmax(float& v, int& i, float& extra) {
#pragma unroll
  for (int o = GROUP / 2; o; o >>= 1) {
    const float ov = __shfl_xor(v, o, GROUP);
    const int oi = __shfl_xor(i, o, GROUP);
    const float oe = __shfl_xor(extra, o, GROUP);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
      extra = oe;
    }
  }
}

// All lanes of the group return the row's action and its log-probability.
// pr may point to global or LDS memory (read only where row_ok and j < A).
__device__ __forceinline__ void draw(const float* pr, int A, bool row_ok, int r, uint32_t k0, uint32_t k1,
                                     float temperature, int j0, int& action, float& log_prob) {
  const bool greedy = !(temperature > 0.f);
  const float div = greedy ? 1.f : temperature;
  float c[MAX_K];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < MAX_K; ++k) {
    const int j = j0 + GROUP * k;
    c[k] = (row_ok && j < A) ? pr[j] / div : -INFINITY;
    mx = fmaxf(mx, c[k]);
  }
  mx = group_max(mx);
  float se = 0.f;
#pragma unroll
  for (int k = 0; k < MAX_K; ++k) se += expf(c[k] - mx);  // exp(-inf) = 0 past A
  float lse = logf(group_sum(se));
  if (greedy) {
    // logits = 0 at argmax(log_softmax(preferences)), -inf elsewhere; their
    // log_softmax is the same vector
    float bv = -INFINITY, dummy = 0.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < MAX_K; ++k) {
      const int j = j0 + GROUP * k;
      const float ls = (c[k] - mx) - lse;
      if (j < A && (ls > bv || bi == 0x7fffffff)) {
        bv = ls;
        bi = j;
      }
    }
    group_argmax(bv, bi, dummy);
#pragma unroll
    for (int k = 0; k < MAX_K; ++k) c[k] = (j0 + GROUP * k == bi) ? 0.f : -INFINITY;
    mx = 0.f;
    lse = 0.f;
  }
  float best = -INFINITY, best_lp = -INFINITY;
  int best_i = 0x7fffffff;
  const uint64_t base = (uint64_t)(row_ok ? r : 0) * (uint64_t)A;
#pragma unroll
  for (int k = 0; k < MAX_K; ++k) {
    const int j = j0 + GROUP * k;
    if (j < A) {
      const float lsm = (c[k] - mx) - lse;
      const float f = ppo::unit_float(ppo::random_word(k0, k1, base + (uint64_t)j));
      // uniform(minval = tiny, maxval = 1): f * (1 - tiny) + tiny, floored at tiny
      const float tiny = 1.17549435e-38f;
      const float u = fmaxf(tiny, f * (1.0f - tiny) + tiny);
      const float z = lsm + -logf(-logf(u));
      if (z > best || best_i == 0x7fffffff) {
        best = z;
        best_i = j;
        best_lp = lsm;
      }
    }
  }
  group_argmax(best, best_i, best_lp);
  action = best_i;
  log_prob = best_lp;
}

}  // namespace cat
}  // namespace ppo
