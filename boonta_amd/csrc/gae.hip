// GAE as a reverse scan over the time-major T x N rollout.
//
// Follows boonta/algorithms/advantage_estimators.py:8-56: for t = T-1 .. 0,
//   delta_t = rho_t * (r_t + gamma * (1 - term_t) * V_{t+1} - V_t) * (1 - trunc_t)
//   A_t     = delta_t + gamma * lambda * c_t * (1 - term_t) * (1 - trunc_t) * A_{t+1}
// with V_T = bootstrap, A_T = 0, and returns_t = A_t + V_t.
//
// Layout: every [T, N] array is time-major, so lane n of a wavefront owns env
// column n and each time step is one coalesced 256-byte row read per wave.
// delta_t depends only on data, so the only serial dependence is the affine
// recurrence A_t = delta_t + k_t A_{t+1}.  When N alone cannot fill the chip,
// the T axis is cut into `chunks` pieces: each piece first folds its steps into
// an affine map (P, Q) with A_start = P + Q * A_after, the maps are chained
// across pieces through LDS, then every piece replays its steps from the true
// carry.  The arithmetic of each step keeps the reference's operation order and
// is not contracted into FMAs.
#include "common.h"

namespace {

struct GaeArgs {
  const float* reward;
  const uint8_t* terminated;
  const uint8_t* truncated;
  const float* values;
  const float* bootstrap;
  const float* rho;  // may be null (1.0)
  const float* c;    // may be null (1.0)
  const float* ratio;  // V-trace: [N, T] importance ratios (row pitch ldr), or null
  int64_t ldr;
  float rho_clip, c_clip;
  float* adv;
  float* ret;
  int T, N;
  float gamma;     // fp32(gamma)
  float gl;        // fp32(gamma * lambda), product taken in double like a Python float
};

struct Step {
  float delta, k;
};

__device__ __forceinline__ Step gae_step(const GaeArgs& a, int t, int n, float next_value) {
  const int64_t i = (int64_t)t * a.N + n;
  const float r = a.reward[i];
  const float te = a.terminated[i] ? 1.f : 0.f;
  const float tr = a.truncated[i] ? 1.f : 0.f;
  const float v = a.values[i];
  float rho = a.rho ? a.rho[i] : 1.f;
  float c = a.c ? a.c[i] : 1.f;
  if (a.ratio) {  // rho = min(ratio, advantage_clip), c = min(ratio, trace_clip)
    // jnp.minimum propagates a NaN ratio (fminf would return the clip value)
    const float q = a.ratio[(int64_t)n * a.ldr + t];
    rho = (q < a.rho_clip || q != q) ? q : a.rho_clip;
    c = (q < a.c_clip || q != q) ? q : a.c_clip;
  }
  const float one_te = __fsub_rn(1.f, te);
  const float one_tr = __fsub_rn(1.f, tr);
  float d = __fadd_rn(r, __fmul_rn(__fmul_rn(a.gamma, one_te), next_value));
  d = __fmul_rn(rho, __fsub_rn(d, v));
  d = __fmul_rn(d, one_tr);
  float k = __fmul_rn(__fmul_rn(__fmul_rn(a.gl, c), one_te), one_tr);
  return {d, k};
}

__device__ __forceinline__ float next_value_at(const GaeArgs& a, int t, int n) {
  // V_{t+1}, with V_T = bootstrap
  return (t + 1 < a.T) ? a.values[(int64_t)(t + 1) * a.N + n] : a.bootstrap[n];
}

// blockDim = (64, chunks): threadIdx.x = column within the wave, threadIdx.y = piece of T.
__global__ void __launch_bounds__(1024) gae_kernel(GaeArgs a) {
  __shared__ float sP[16][64];
  __shared__ float sQ[16][64];
  const int n = blockIdx.x * 64 + threadIdx.x;
  const int chunks = blockDim.y;
  const int j = threadIdx.y;
  const bool live = n < a.N;
  const int t_lo = (int)(((int64_t)a.T * j) / chunks);
  const int t_hi = (int)(((int64_t)a.T * (j + 1)) / chunks);  // exclusive

  float carry = 0.f;
  if (chunks > 1) {
    float P = 0.f, Q = 1.f;
    if (live) {
      for (int t = t_hi - 1; t >= t_lo; --t) {
        Step s = gae_step(a, t, n, next_value_at(a, t, n));
        P = __fadd_rn(s.delta, __fmul_rn(s.k, P));
        Q = __fmul_rn(s.k, Q);
      }
    }
    sP[j][threadIdx.x] = P;
    sQ[j][threadIdx.x] = Q;
    __syncthreads();
    for (int q = chunks - 1; q > j; --q)
      carry = __fadd_rn(sP[q][threadIdx.x], __fmul_rn(sQ[q][threadIdx.x], carry));
  }
  if (!live) return;
  float A = carry;
  for (int t = t_hi - 1; t >= t_lo; --t) {
    const float nv = next_value_at(a, t, n);
    Step s = gae_step(a, t, n, nv);
    A = __fadd_rn(s.delta, __fmul_rn(s.k, A));
    const int64_t i = (int64_t)t * a.N + n;
    a.adv[i] = A;
    a.ret[i] = __fadd_rn(A, a.values[i]);
  }
}

}  // namespace

namespace {

int launch_gae(void* stream, GaeArgs a, double gamma, double gae_lambda, int chunks, const char* name) {
  const int T = a.T, N = a.N;
  if (T < 0 || N < 0) return ppo::set_error(PPO_ERR_ARG, "%s: negative shape T=%d N=%d", name, T, N);
  if (T == 0 || N == 0) return PPO_OK;
  if (!a.reward || !a.terminated || !a.truncated || !a.values || !a.bootstrap || !a.adv || !a.ret)
    return ppo::set_error(PPO_ERR_ARG, "%s: null buffer", name);
  if (chunks <= 0) {
    // enough waves for ~4 per CU, capped by T and the LDS table
    const int waves = (N + 63) / 64;
    chunks = 1;
    while (chunks < 16 && waves * chunks < 1024 && T / (chunks * 2) >= 4) chunks *= 2;
  }
  if (chunks > 16) return ppo::set_error(PPO_ERR_ARG, "%s: chunks %d > 16", name, chunks);
  if (chunks > T) chunks = T;
  a.gamma = (float)gamma;
  a.gl = (float)(gamma * gae_lambda);
  dim3 block(64, chunks);
  dim3 grid((N + 63) / 64);
  hipLaunchKernelGGL(gae_kernel, grid, block, 0, ppo::as_stream(stream), a);
  return ppo::check_launch(name);
}

}  // namespace

PPO_EXPORT int ppo_gae_f32(void* stream, const float* reward, const uint8_t* terminated,
                           const uint8_t* truncated, const float* values,
                           const float* bootstrap, const float* rho, const float* c,
                           float* advantages, float* returns, int T, int N, double gamma,
                           double gae_lambda, int chunks) {
  GaeArgs a{reward, terminated, truncated, values, bootstrap, rho, c, nullptr, 0, 0.f, 0.f, advantages, returns,
            T, N, 0.f, 0.f};
  return launch_gae(stream, a, gamma, gae_lambda, chunks, "ppo_gae_f32");
}

// V-trace as RecurrentPuPO.update calls the estimator
// (boonta/algorithms/recurrent_pupo.py:210-220): ratio is [N, T] (env-major,
// row pitch ldr) and rho = min(ratio, advantage_clip), c = min(ratio,
// trace_clip) are formed as the scan reads them.
PPO_EXPORT int ppo_vtrace_f32(void* stream, const float* reward, const uint8_t* terminated,
                              const uint8_t* truncated, const float* values, const float* bootstrap,
                              const float* ratio, int64_t ldr, float advantage_clip, float trace_clip,
                              float* advantages, float* returns, int T, int N, double gamma, double gae_lambda,
                              int chunks) {
  if (!ratio || ldr < T)
    return ppo::set_error(PPO_ERR_ARG, "ppo_vtrace_f32: ratio [N, T] needs a row pitch >= T (%lld < %d)",
                          (long long)ldr, T);
  GaeArgs a{reward, terminated, truncated, values, bootstrap, nullptr, nullptr, ratio, ldr, advantage_clip,
            trace_clip, advantages, returns, T, N, 0.f, 0.f};
  return launch_gae(stream, a, gamma, gae_lambda, chunks, "ppo_vtrace_f32");
}

// ------------------------------------------------- advantage normalisation
// (A - mean(A)) / (std(A) + 1e-8) over all T * N advantages, population
// std, as boonta/algorithms/ppo.py:220-221 (recurrent_ppo.py:206-207).  Three
// launches without a grid barrier: per-block sums; every block folds the sums
// into the mean and writes per-block sums of squared deviations; every block
// folds those into the std and normalises its elements.  Partial sums are
// fp64 and folded in a fixed order.
namespace {

constexpr int NORM_THREADS = 256;
constexpr int NORM_PER_THREAD = 16;
constexpr int NORM_PER_BLOCK = NORM_THREADS * NORM_PER_THREAD;

// sum over a workgroup of THREADS threads; every thread gets the total
template <int THREADS = NORM_THREADS>
__device__ double block_sum_d(double v) {
  __shared__ double s[THREADS / 64];
  v = ppo::wave_sum_d(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) s[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < THREADS / 64; ++i) t += s[i];
  __syncthreads();
  return t;
}

__device__ double fold(const double* part, int nblocks) {
  // every thread folds the same partials in the same order
  double t = 0.0;
  for (int i = 0; i < nblocks; ++i) t += part[i];
  return t;
}

__global__ void __launch_bounds__(NORM_THREADS) norm_sum_kernel(const float* a, int64_t n, double* part) {
  const int64_t base = (int64_t)blockIdx.x * NORM_PER_BLOCK;
  double v = 0.0;
  for (int j = 0; j < NORM_PER_THREAD; ++j) {
    const int64_t i = base + (int64_t)j * NORM_THREADS + threadIdx.x;
    if (i < n) v += (double)a[i];
  }
  v = block_sum_d(v);
  if (threadIdx.x == 0) part[blockIdx.x] = v;
}

__global__ void __launch_bounds__(NORM_THREADS) norm_dev_kernel(const float* a, int64_t n, const double* sums,
                                                                double* part, int nblocks) {
  const double mean = fold(sums, nblocks) / (double)n;
  const int64_t base = (int64_t)blockIdx.x * NORM_PER_BLOCK;
  double v = 0.0;
  for (int j = 0; j < NORM_PER_THREAD; ++j) {
    const int64_t i = base + (int64_t)j * NORM_THREADS + threadIdx.x;
    if (i < n) {
      const double d = (double)a[i] - mean;
      v += d * d;
    }
  }
  v = block_sum_d(v);
  if (threadIdx.x == 0) part[blockIdx.x] = v;
}

__global__ void __launch_bounds__(NORM_THREADS) norm_apply_kernel(float* a, int64_t n, const double* sums,
                                                                  const double* devs, int nblocks) {
  const float mean = (float)(fold(sums, nblocks) / (double)n);
  const float stdv = (float)sqrt(fold(devs, nblocks) / (double)n);
  const float den = stdv + 1e-8f;
  const int64_t base = (int64_t)blockIdx.x * NORM_PER_BLOCK;
  for (int j = 0; j < NORM_PER_THREAD; ++j) {
    const int64_t i = base + (int64_t)j * NORM_THREADS + threadIdx.x;
    if (i < n) a[i] = (a[i] - mean) / den;
  }
}

// RecurrentPuPO's minibatch advantages (boonta/algorithms/recurrent_pupo.py
// :244-250), one workgroup: the V-trace advantages of the minibatch's samples
// rows[i] (t * N + env, listed time-major: row t * width + b), normalised over
// the minibatch when `normalize` ((A - mean) / (std + 1e-8), population std,
// sums in float64), times the importance weight of the row's sequence b:
//   out[rows[i]] = weights[i % width] * A'[i].
// A sequence drawn twice (choice with replacement) writes the same value
// twice: its samples, weight and the minibatch statistics are the same.
constexpr int PUPO_THREADS = 1024;

__global__ void __launch_bounds__(PUPO_THREADS) pupo_advantages_kernel(const float* adv, const int32_t* rows,
                                                                       int count, const float* weights, int width,
                                                                       int normalize, float* out) {
  float mean = 0.f, den = 1.f;
  if (normalize) {
    double v = 0.0;
    for (int i = threadIdx.x; i < count; i += PUPO_THREADS) v += (double)adv[rows[i]];
    const double m = block_sum_d<PUPO_THREADS>(v) / (double)count;
    double d2 = 0.0;
    for (int i = threadIdx.x; i < count; i += PUPO_THREADS) {
      const double d = (double)adv[rows[i]] - m;
      d2 += d * d;
    }
    const double var = block_sum_d<PUPO_THREADS>(d2) / (double)count;
    mean = (float)m;
    den = (float)sqrt(var) + 1e-8f;
  }
  for (int i = threadIdx.x; i < count; i += PUPO_THREADS) {
    const int32_t r = rows[i];
    const float a = normalize ? (adv[r] - mean) / den : adv[r];
    out[r] = weights[i % width] * a;
  }
}

__global__ void fill_kernel(float* a, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) a[i] = v;
}

}  // namespace

PPO_EXPORT int ppo_pupo_advantages_f32(void* stream, const float* adv, const int32_t* rows, int count,
                                       const float* weights, int width, int normalize, float* out) {
  if (count < 0 || width < 1 || (count > 0 && count % width))
    return ppo::set_error(PPO_ERR_ARG, "ppo_pupo_advantages_f32: %d rows are not whole steps of %d sequences",
                          count, width);
  if (count == 0) return PPO_OK;
  if (!adv || !rows || !weights || !out) return ppo::set_error(PPO_ERR_ARG, "ppo_pupo_advantages_f32: null buffer");
  hipLaunchKernelGGL(pupo_advantages_kernel, dim3(1), dim3(PUPO_THREADS), 0, ppo::as_stream(stream), adv, rows, count,
                     weights, width, normalize, out);
  return ppo::check_launch("ppo_pupo_advantages_f32");
}

PPO_EXPORT int ppo_fill_f32(void* stream, float* a, int64_t n, float value) {
  if (n < 0 || (n > 0 && !a)) return ppo::set_error(PPO_ERR_ARG, "ppo_fill_f32: bad argument");
  if (n == 0) return PPO_OK;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)ppo::ceil_div64(n, 256)), dim3(256), 0, ppo::as_stream(stream), a, n,
                     value);
  return ppo::check_launch("ppo_fill_f32");
}

PPO_EXPORT size_t ppo_normalize_workspace(int64_t n) {
  if (n <= 0) return 0;
  return 2 * sizeof(double) * (size_t)ppo::ceil_div64(n, NORM_PER_BLOCK);
}

PPO_EXPORT int ppo_normalize_advantages_f32(void* stream, float* adv, int64_t n, void* workspace,
                                            size_t workspace_bytes) {
  if (n < 0) return ppo::set_error(PPO_ERR_ARG, "ppo_normalize_advantages_f32: negative size");
  if (n == 0) return PPO_OK;
  if (!adv || !workspace) return ppo::set_error(PPO_ERR_ARG, "ppo_normalize_advantages_f32: null buffer");
  if (workspace_bytes < ppo_normalize_workspace(n))
    return ppo::set_error(PPO_ERR_SPACE, "ppo_normalize_advantages_f32: workspace %zu < %zu bytes",
                          workspace_bytes, ppo_normalize_workspace(n));
  const int64_t nb = ppo::ceil_div64(n, NORM_PER_BLOCK);
  if (nb > (1 << 20)) return ppo::set_error(PPO_ERR_ARG, "ppo_normalize_advantages_f32: n too large");
  double* sums = static_cast<double*>(workspace);
  double* devs = sums + nb;
  hipStream_t s = ppo::as_stream(stream);
  hipLaunchKernelGGL(norm_sum_kernel, dim3((unsigned)nb), dim3(NORM_THREADS), 0, s, adv, n, sums);
  hipLaunchKernelGGL(norm_dev_kernel, dim3((unsigned)nb), dim3(NORM_THREADS), 0, s, adv, n, sums, devs, (int)nb);
  hipLaunchKernelGGL(norm_apply_kernel, dim3((unsigned)nb), dim3(NORM_THREADS), 0, s, adv, n, sums, devs, (int)nb);
  return ppo::check_launch("ppo_normalize_advantages_f32");
}
