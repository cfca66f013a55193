// Action sampling of the rollout-side PPO.step (boonta/algorithms/ppo.py:57-74):
// dist.sample_and_log_prob(seed=key) on the network's head outputs, plus the
// value column copied out (remove_feature_axis, utils/axis.py:11-12).
//
// Categorical (boonta/networks/distributions.py:8-23, distrax 0.1.9):
//   cooled  = preferences / (T if T > 0 else 1); at T <= 0 the logits are 0 at
//             argmax(log_softmax(preferences)) and -inf elsewhere
//   logits  = log_softmax(cooled)                        (distrax normalises)
//   action  = argmax(logits + gumbel(key, (1, rows, A))) (first index on ties)
//   log_prob = logits[action]
// with gumbel = -log(-log(u)), u = uniform(key, shape, minval=tiny, maxval=1)
// (jax.random.gumbel, low-dynamic-range mode).
//
// Diagonal Gaussian (distributions.py:42-57: MultivariateNormalDiag(mean, sigma),
// sigma = T * (softplus(s) + 1e-3)), sampled through distrax's bijector form:
//   eps = normal(key, (1, rows, D)) = sqrt(2) * erfinv(u),
//         u = uniform(key, shape, minval=nextafter(-1, 0), maxval=1)
//   action   = sigma * eps + mean
//   log_prob = sum_d(-eps^2 / 2 - log(2 pi) / 2) - sum_d log sigma
//
// The uniform draws follow jax.random.uniform: word i of the key's 32-bit
// stream (threefry.h), its top 23 bits as the mantissa of a float in [1, 2),
// minus 1, scaled by (maxval - minval) in float32, plus minval, floored at
// minval.  erfinv is M. Giles' single-precision approximation ("Approximating
// the erfinv function", GPU Computing Gems Jade Edition, 2011), the form XLA
// lowers float32 erf_inv to.
//
// Layout: one 16-lane group of a wave per row, lane j owning columns j, j + 16,
// ...; row statistics (max, sum, argmax, log-prob sum) are 16-lane butterflies.
#include "common.h"
#include "threefry.h"
#include "categorical.h"

#include <math.h>

namespace {

constexpr int GROUP = 16;
constexpr int THREADS = 256;
constexpr int ROWS_PER_BLOCK = THREADS / GROUP;
constexpr int MAX_K = 8;  // columns per lane: A, D <= 128
constexpr float HALF_LOG_2PI = 0.91893853320467274f;

__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = GROUP / 2; o; o >>= 1) v += __shfl_xor(v, o, GROUP);
  return v;
}

__device__ __forceinline__ float softplus_acc(float x) {
  // jax.nn.softplus = logaddexp(x, 0)
  return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x)));
}

__device__ __forceinline__ float erfinv_giles(float x) {
  float w = -log1pf(-(x * x));
  float p;
  if (w < 5.0f) {
    w = w - 2.5f;
    p = 2.81022636e-08f;
    p = 3.43273939e-07f + p * w;
    p = -3.5233877e-06f + p * w;
    p = -4.39150654e-06f + p * w;
    p = 0.00021858087f + p * w;
    p = -0.00125372503f + p * w;
    p = -0.00417768164f + p * w;
    p = 0.246640727f + p * w;
    p = 1.50140941f + p * w;
  } else {
    w = sqrtf(w) - 3.0f;
    p = -0.000200214257f;
    p = 0.000100950558f + p * w;
    p = 0.00134934322f + p * w;
    p = -0.00367342844f + p * w;
    p = 0.00573950773f + p * w;
    p = -0.0076224613f + p * w;
    p = 0.00943887047f + p * w;
    p = 1.00167406f + p * w;
    p = 2.83297682f + p * w;
  }
  return fabsf(x) == 1.0f ? x * INFINITY : p * x;
}

struct CatArgs {
  const float* pref;
  int64_t ldp;
  int rows, A;
  const float* vsrc;
  int64_t ldv;
  const uint32_t* key;
  float temperature;
  int32_t* action;
  float* log_prob;
  float* value;
};

__global__ void __launch_bounds__(THREADS) sample_categorical_kernel(CatArgs a) {
  const int r = blockIdx.x * ROWS_PER_BLOCK + (int)(threadIdx.x / GROUP);
  const int j0 = threadIdx.x % GROUP;
  const bool row_ok = r < a.rows;
  const uint32_t k0 = a.key[0], k1 = a.key[1];
  const float* pr = a.pref + (int64_t)(row_ok ? r : 0) * a.ldp;
  int act_i;
  float lp;
  ppo::cat::draw(pr, a.A, row_ok, r, k0, k1, a.temperature, j0, act_i, lp);
  if (row_ok && j0 == 0) {
    a.action[r] = act_i;
    a.log_prob[r] = lp;
    if (a.value) a.value[r] = a.vsrc[(int64_t)r * a.ldv];
  }
}

struct GaussArgs {
  const float* mean;
  int64_t ldm;
  const float* scale;  // raw scale s: [rows, lds] per row, or [D] when lds == 0
  int64_t lds;
  int rows, D;
  const float* vsrc;
  int64_t ldv;
  const uint32_t* key;
  float temperature;
  float* action;
  int64_t lda;
  float* log_prob;
  float* value;
};

__global__ void __launch_bounds__(THREADS) sample_gaussian_kernel(GaussArgs a) {
  const int r = blockIdx.x * ROWS_PER_BLOCK + (int)(threadIdx.x / GROUP);
  const int j0 = threadIdx.x % GROUP;
  const bool row_ok = r < a.rows;
  const uint32_t k0 = a.key[0], k1 = a.key[1];
  const float lo = -0.99999994f;  // nextafter(-1, 0)
  const float span = 1.0f - lo;   // maxval - minval, rounded to float32
  const uint64_t base = (uint64_t)(row_ok ? r : 0) * (uint64_t)a.D;
  float lpx = 0.f, logdet = 0.f;
#pragma unroll
  for (int k = 0; k < MAX_K; ++k) {
    const int j = j0 + GROUP * k;
    if (row_ok && j < a.D) {
      const float f = ppo::unit_float(ppo::random_word(k0, k1, base + (uint64_t)j));
      const float u = fmaxf(lo, f * span + lo);
      const float eps = 1.41421356237309515f * erfinv_giles(u);
      const float raw = a.lds ? a.scale[(int64_t)r * a.lds + j] : a.scale[j];
      const float sig = a.temperature * (softplus_acc(raw) + 1e-3f);
      a.action[(int64_t)r * a.lda + j] = sig * eps + a.mean[(int64_t)r * a.ldm + j];
      lpx += -0.5f * (eps * eps) - HALF_LOG_2PI;
      logdet += logf(sig);
    }
  }
  lpx = group_sum(lpx);
  logdet = group_sum(logdet);
  if (row_ok && j0 == 0) {
    a.log_prob[r] = lpx - logdet;
    if (a.value) a.value[r] = a.vsrc[(int64_t)r * a.ldv];
  }
}

}  // namespace

PPO_EXPORT int ppo_sample_max_outputs() { return GROUP * MAX_K; }

PPO_EXPORT int ppo_sample_categorical_f32(void* stream, const float* pref, int64_t ldp, int rows, int A,
                                          const float* value_src, int64_t ldv, const uint32_t* key,
                                          float temperature, int32_t* action, float* log_prob, float* value) {
  if (rows < 0 || A < 1 || A > GROUP * MAX_K || ldp < A || !pref || !key || !action || !log_prob ||
      (value && (!value_src || ldv < 1)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_sample_categorical_f32: bad argument (rows %d, A %d, ldp %lld)", rows,
                          A, (long long)ldp);
  if (rows == 0) return PPO_OK;
  CatArgs a{pref, ldp, rows, A, value_src, ldv, key, temperature, action, log_prob, value};
  hipLaunchKernelGGL(sample_categorical_kernel, dim3(ppo::ceil_div(rows, ROWS_PER_BLOCK)), dim3(THREADS), 0,
                     ppo::as_stream(stream), a);
  return ppo::check_launch("ppo_sample_categorical_f32");
}

PPO_EXPORT int ppo_sample_gaussian_f32(void* stream, const float* mean, int64_t ldm, const float* scale_raw,
                                       int64_t lds, int rows, int D, const float* value_src, int64_t ldv,
                                       const uint32_t* key, float temperature, float* action, int64_t lda,
                                       float* log_prob, float* value) {
  if (rows < 0 || D < 1 || D > GROUP * MAX_K || ldm < D || lda < D || lds < 0 || (lds > 0 && lds < D) || !mean ||
      !scale_raw || !key || !action || !log_prob || (value && (!value_src || ldv < 1)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_sample_gaussian_f32: bad argument (rows %d, D %d)", rows, D);
  if (rows == 0) return PPO_OK;
  GaussArgs a{mean, ldm, scale_raw, lds, rows, D, value_src, ldv, key, temperature, action, lda, log_prob, value};
  hipLaunchKernelGGL(sample_gaussian_kernel, dim3(ppo::ceil_div(rows, ROWS_PER_BLOCK)), dim3(THREADS), 0,
                     ppo::as_stream(stream), a);
  return ppo::check_launch("ppo_sample_gaussian_f32");
}
