// Prioritised minibatch selection of RecurrentPuPO.update
// (boonta/algorithms/recurrent_pupo.py:226-236), one launch per minibatch:
//
//   priority[n]  = (sum_t |A[t, n]|) ** priority_exponent     A: [T, N] V-trace
//   prob[n]      = (priority[n] + 1e-6) / (sum_n priority[n] + 1e-6)
//   idx          = jax.random.choice(key, N, (width,), replace=True, p=prob)
//   weight[i]    = (N * prob[idx[i]]) ** -beta
//
// jax.random.choice with replace=True and p (jax/_src/random.py, jax 0.10.2)
// draws through the inverse CDF: c = cumsum(p); r = c[N-1] * (1 - u) with
// u = uniform(key, (width,)) (word i of the key's Threefry stream, threefry.h);
// idx = searchsorted(c, r), the first n with c[n] >= r.
//
// One workgroup of 1024 threads: the per-env sums over T read coalesced rows
// of A (consecutive threads, consecutive envs) in float32, t in order; the
// probabilities are float32 as the reference forms them; their running sum is
// taken in float64 in LDS (N <= 16384: 128 KB of the 160 KB), a per-thread
// run over a contiguous block of envs plus a workgroup scan of the run
// totals, and each draw is a binary search of it.  XLA's float32 cumsum
// rounds differently: an index can differ from the reference's only where r
// falls within float32 rounding of a cumulative boundary.  Measured against a
// float32 sequential cumsum with float32 r: no index differs at 1024 envs
// drawing 256; at most 0.6 % of draws move to a neighbouring env up to 16384
// envs.
#include "common.h"
#include "threefry.h"

#include <math.h>

namespace {

constexpr int PC_THREADS = 1024;
constexpr int PC_MAX_ENVS = 16384;

struct PriorityArgs {
  const float* adv;
  int64_t lda;
  int T, N;
  float exponent, beta;
  const uint32_t* key;
  int width;
  int32_t* indices;
  float* weights;
  float* probabilities;
};

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// (sum_t |A[t, n]|) ** exponent in float32, t in order (eight loads in
// flight before their adds)
__device__ __forceinline__ float env_priority(const PriorityArgs& a, int n) {
  const float* col = a.adv + n;
  float s = 0.f;
  int t = 0;
  for (; t + 8 <= a.T; t += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = col[(int64_t)(t + j) * a.lda];
#pragma unroll
    for (int j = 0; j < 8; ++j) s += fabsf(v[j]);
  }
  for (; t < a.T; ++t) s += fabsf(col[(int64_t)t * a.lda]);
  return powf(s, a.exponent);
}

__global__ void __launch_bounds__(PC_THREADS) priority_choice_kernel(PriorityArgs a) {
  __shared__ double cum[PC_MAX_ENVS];
  __shared__ double wtot[PC_THREADS / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int N = a.N;

  // priority per env; its total over the workgroup
  double part = 0.0;
  for (int n = tid; n < N; n += PC_THREADS) {
    const float pr = env_priority(a, n);
    cum[n] = pr;
    part += pr;
  }
  part = wave_sum(part);
  if (lane == 0) wtot[wave] = part;
  __syncthreads();
  double total = 0.0;
#pragma unroll
  for (int w = 0; w < PC_THREADS / 64; ++w) total += wtot[w];
  const float denom = (float)total + 1e-6f;
  __syncthreads();  // wtot is reused by the scan

  // float32 probabilities, then their inclusive running sum in float64:
  // thread tid owns the contiguous envs [tid * per, tid * per + per)
  const int per = (N + PC_THREADS - 1) / PC_THREADS;
  const int b0 = min(tid * per, N), b1 = min(b0 + per, N);
  double run = 0.0;
  for (int n = b0; n < b1; ++n) {
    const float pn = ((float)cum[n] + 1e-6f) / denom;
    a.probabilities[n] = pn;
    run += pn;
    cum[n] = run;  // local inclusive sums, offset added below
  }
  // exclusive scan of the run totals across the workgroup
  double inc = run;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double y = __shfl_up(inc, o, 64);
    if (lane >= o) inc += y;
  }
  if (lane == 63) wtot[wave] = inc;
  __syncthreads();
  double off = inc - run;
  for (int w = 0; w < wave; ++w) off += wtot[w];
  for (int n = b0; n < b1; ++n) cum[n] += off;
  __syncthreads();

  // draws: r = c[N-1] * (1 - u), idx = first n with c[n] >= r
  const double last = cum[N - 1];
  const uint32_t k0 = a.key[0], k1 = a.key[1];
  for (int i = tid; i < a.width; i += PC_THREADS) {
    const float u = ppo::unit_float(ppo::random_word(k0, k1, (uint64_t)i));
    const double r = last * (double)(1.0f - u);  // 1 - u is exact in float32
    int lo = 0, hi = N;  // searchsorted(side='left') over [0, N]
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cum[mid] < r) lo = mid + 1; else hi = mid;
    }
    const int idx = min(lo, N - 1);
    a.indices[i] = idx;
    // probabilities[idx], recomputed with the same float32 operations
    const float p_idx = (env_priority(a, idx) + 1e-6f) / denom;
    a.weights[i] = powf((float)N * p_idx, -a.beta);
  }
}

}  // namespace

PPO_EXPORT int ppo_priority_choice_max_envs() { return PC_MAX_ENVS; }

PPO_EXPORT int ppo_priority_choice_f32(void* stream, const float* advantages, int64_t lda, int T, int N,
                                       float priority_exponent, float beta, const uint32_t* key, int width,
                                       int32_t* indices, float* weights, float* probabilities) {
  if (T < 1 || N < 1 || N > PC_MAX_ENVS || lda < N || width < 0 || !advantages || !key || !probabilities ||
      (width > 0 && (!indices || !weights)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_priority_choice_f32: bad argument (T %d, N %d, width %d; N <= %d)", T, N,
                          width, PC_MAX_ENVS);
  PriorityArgs a{advantages, lda, T, N, priority_exponent, beta, key, width, indices, weights, probabilities};
  hipLaunchKernelGGL(priority_choice_kernel, dim3(1), dim3(PC_THREADS), 0, ppo::as_stream(stream), a);
  return ppo::check_launch("ppo_priority_choice_f32");
}
