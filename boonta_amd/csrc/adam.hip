// Gradient assembly and the optimizer step of the learner:
//
//   1. ppo_grad_reduce: every gradient leaf arrives as `nparts` partial
//      buffers (split-K GEMM slices, per-block LayerNorm / scale partials).
//      One launch sums them in a fixed order straight into the flat gradient
//      buffer and leaves one partial sum of squares per block for the norm.
//   2. ppo_adam_clip_f32: optax.chain(clip_by_global_norm(max_norm), adam(lr))
//      of optax 0.2.8, as every PPO recipe builds it
//      (hangar/recipes/ppo_cartpole.py:44-47; applied at
//      boonta/algorithms/ppo.py:182-191) in one bandwidth-bound pass over the
//      flat parameter, gradient and moment buffers:
//        g <- g                      if ||g|| < max_norm
//             (g / ||g||) * max_norm otherwise
//        mu = (1-b1) g + b1 mu;  nu = (1-b2) g^2 + b2 nu;  count += 1
//        p  <- p + (-lr) * ((mu / (1 - b1^count)) / (sqrt(nu / (1 - b2^count)) + eps))
//      The global norm is re-folded from the per-block partials by every
//      block, so no extra launch or grid barrier is needed, and the optax
//      step counter lives in device memory (count_base + step_offset + 1), so
//      a captured graph replays with the right bias corrections.
#include "grad_reduce.h"

#include <algorithm>

namespace {

using ppo_gr::Chunk;
using ppo_gr::Segment;
using ppo_gr::CHUNK;
using ppo_gr::FEW_PARTS;
using ppo_gr::REDUCE_THREADS;
using ppo_gr::WIDE_CHUNK;
using ppo_gr::WIDE_PARTS;

// One block per chunk (ppo_gr::reduce_block: the fixed-order sum, the
// summed values written to the flat gradient, one squared-norm partial per
// chunk).
__global__ void __launch_bounds__(REDUCE_THREADS)
grad_reduce_kernel(const Segment* __restrict__ segs, const Chunk* __restrict__ chunks, int nchunks, int nfew,
                   int nwide, double* __restrict__ sumsq) {
  __shared__ floatx4 part[REDUCE_THREADS / 64][64];
  ppo_gr::reduce_block((int)blockIdx.x, segs, chunks, nchunks, nfew, nwide, sumsq, part);
}

constexpr int ADAM_TR_MAX = 8;

struct AdamParams {
  float* p;
  const float* g;
  float* mu;
  float* nu;
  void* p_bf16;    // optional bf16 image of the parameters (16-bit patterns)
  int64_t n;       // multiple of 4
  const double* sumsq;
  int nsumsq;
  float max_norm;  // <= 0: no clipping
  float neg_lr;    // fp32(-lr)
  float b1, b2;    // fp32(b1), fp32(b2): the decay of the old moment and of the bias correction
  float omb1, omb2;  // fp32(1 - b1), fp32(1 - b2) with the difference taken in double
  float eps;
  const int* count_base;
  int step_offset;
  const int* abort_word;  // may be null; nonzero: the step is skipped (nothing written)
  // 256 x 256 kernels (row-major, at element offset tr_off[r] of p) whose
  // updated values are also written transposed to tr_dst[r] ([256][256]):
  // blocks from plain_blocks on update them a few rows at a time, and the
  // grid-stride pass of the other blocks skips them
  int ntr;
  int plain_blocks;
  int64_t tr_off[ADAM_TR_MAX];
  float* tr_dst[ADAM_TR_MAX];
};

// One element group's Adam step (and its bf16 image) in place.  Every
// product and sum is rounded on its own (no fused multiply-add), so the step
// is the same bits in each kernel that inlines it.
__device__ __forceinline__ void adam_update(const AdamParams& a, int64_t i, floatx4 g, floatx4& m, floatx4& v,
                                            floatx4& p, float norm, bool clip, float bc1, float bc2) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float ge = g[e];
    if (clip) ge = (ge / norm) * a.max_norm;
    const float me = a.omb1 * ge + a.b1 * m[e];
    const float ve = a.omb2 * (ge * ge) + a.b2 * v[e];
    m[e] = me;
    v[e] = ve;
    const float u = a.neg_lr * ((me / bc1) / (sqrtf(ve / bc2) + a.eps));
    p[e] = p[e] + u;
  }
  reinterpret_cast<floatx4*>(a.mu)[i] = m;
  reinterpret_cast<floatx4*>(a.nu)[i] = v;
  reinterpret_cast<floatx4*>(a.p)[i] = p;
  if (a.p_bf16) {
    // the bf16 image a bf16-compute layer multiplies with (round to nearest even)
    uint2 b;
    b.x = ppo::bf16_bits(p[0]) | (ppo::bf16_bits(p[1]) << 16);
    b.y = ppo::bf16_bits(p[2]) | (ppo::bf16_bits(p[3]) << 16);
    reinterpret_cast<uint2*>(a.p_bf16)[i] = b;
  }
}

// The j-th element group (float4 index) outside the transposed kernels
// (their offsets ascending).
__device__ __forceinline__ int64_t plain_index(const AdamParams& a, int64_t j) {
  int64_t i = j;
#pragma unroll
  for (int r = 0; r < ADAM_TR_MAX; ++r)
    if (r < a.ntr && i >= a.tr_off[r] / 4) i += 256 * 256 / 4;
  return i;
}

// Rows of a transposed kernel per job: one element group per thread, as in
// the grid-stride pass (more rows per job made those blocks the launch's
// tail).
constexpr int TJ_ROWS = 4;
static_assert(TJ_ROWS * 8 == 32, "eight jobs fill a 32-row group");
constexpr int TJ_G = TJ_ROWS / 4;  // element groups per thread

// WT: the launch also runs transposed-kernel jobs (ppo_adam_clip_wt_f32); the
// plain launch keeps the registers and LDS of the grid-stride pass alone.
template <bool WT>
__global__ void __launch_bounds__(256) adam_kernel(AdamParams a) {
  __shared__ float s_scale_norm[2];
  __shared__ float s_bc[2];
  __shared__ int s_abort;
  __shared__ double s_w[4];
  __shared__ float s_tile[WT ? TJ_ROWS : 1][256 + 4];  // a transposed kernel job's updated rows
  // the grid-stride pass runs over the element groups outside the
  // transposed kernels: j < n4 of them, group plain_index(j)
  const int64_t n4 = a.n / 4 - (WT ? (int64_t)a.ntr * (256 * 256 / 4) : 0);
  const bool tjob = WT && (int)blockIdx.x >= a.plain_blocks;
  const int64_t stride = (int64_t)a.plain_blocks * blockDim.x;
  int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t i = WT ? plain_index(a, j) : j;
  // a transposed kernel job: TJ_ROWS rows of kernel r; thread t owns element
  // group c = t % 64 of rows row0 + t / 64 + 4 j (j < TJ_G).  The eight jobs
  // of one 32-row group (whose transposed rows share 128-byte lines) are
  // placed 8 blocks apart, on one XCD (blocks are dealt to the 8 XCDs in
  // turn and plain_blocks is a multiple of 8), so every line of the image is
  // completed in one L2.
  const int job = (int)blockIdx.x - a.plain_blocks;
  const int grp = (job & 7) + 8 * ((job >> 3) >> 3);  // 32-row group over all kernels
  const int tr = tjob ? grp >> 3 : 0;
  const int row0 = tjob ? 32 * (grp & 7) + TJ_ROWS * ((job >> 3) & 7) : 0;
  int64_t ti[TJ_G];
  floatx4 tg[TJ_G], tm[TJ_G], tv[TJ_G], tp[TJ_G];
  if (tjob) {
    int64_t off = 0;
#pragma unroll
    for (int r = 0; r < ADAM_TR_MAX; ++r)
      if (r == tr) off = a.tr_off[r];
#pragma unroll
    for (int j = 0; j < TJ_G; ++j) {
      ti[j] = off / 4 + (int64_t)(row0 + (int)(threadIdx.x >> 6) + 4 * j) * 64 + (threadIdx.x & 63);
      tg[j] = reinterpret_cast<const floatx4*>(a.g)[ti[j]];
      tm[j] = reinterpret_cast<floatx4*>(a.mu)[ti[j]];
      tv[j] = reinterpret_cast<floatx4*>(a.nu)[ti[j]];
      tp[j] = reinterpret_cast<floatx4*>(a.p)[ti[j]];
    }
  }
  // the first group's loads go out with the norm partials' loads below, so
  // the two round trips overlap
  floatx4 g, m, v, p;
  if (!tjob && j < n4) {
    g = reinterpret_cast<const floatx4*>(a.g)[i];
    m = reinterpret_cast<floatx4*>(a.mu)[i];
    v = reinterpret_cast<floatx4*>(a.nu)[i];
    p = reinterpret_cast<floatx4*>(a.p)[i];
  }
  // the squared norm from its partials, in a fixed order every block repeats:
  // thread t adds partials t, t + 256, ..., then wave sums, then the four
  // wave totals in wave order
  {
    double t = ppo::strided_sum_d<256, 4>(a.sumsq, a.nsumsq, threadIdx.x);
    t = ppo::wave_sum_d(t);
    if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = t;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const double t = (s_w[0] + s_w[1]) + (s_w[2] + s_w[3]);
    if (threadIdx.x == 0) {
      const float norm = (float)sqrt(t);
      s_scale_norm[0] = norm;
      s_scale_norm[1] = (a.max_norm > 0.f && !(norm < a.max_norm)) ? 1.f : 0.f;
      const int count = *a.count_base + a.step_offset + 1;
      s_bc[0] = 1.f - powf(a.b1, (float)count);
      s_bc[1] = 1.f - powf(a.b2, (float)count);
      s_abort = a.abort_word ? *a.abort_word : 0;
    }
  }
  __syncthreads();
  // an earlier launch of this update flagged its results unusable: leave the
  // parameters and moments as they are
  if (s_abort != 0) return;
  const float norm = s_scale_norm[0];
  const bool clip = s_scale_norm[1] != 0.f;
  const float bc1 = s_bc[0], bc2 = s_bc[1];
  if constexpr (WT) {
    if (tjob) {
      const int c = threadIdx.x & 63;
#pragma unroll
      for (int j = 0; j < TJ_G; ++j) {
        adam_update(a, ti[j], tg[j], tm[j], tv[j], tp[j], norm, clip, bc1, bc2);
        *reinterpret_cast<floatx4*>(&s_tile[(threadIdx.x >> 6) + 4 * j][4 * c]) = tp[j];
      }
      __syncthreads();
      // thread o writes row o of the transposed image: columns row0 .. row0 + TJ_ROWS - 1
      float* dst = nullptr;
#pragma unroll
      for (int r = 0; r < ADAM_TR_MAX; ++r)
        if (r == tr) dst = a.tr_dst[r];
      const int o = threadIdx.x;
#pragma unroll
      for (int j = 0; j < TJ_G; ++j)
        *reinterpret_cast<floatx4*>(dst + (int64_t)o * 256 + row0 + 4 * j) =
            floatx4{s_tile[4 * j][o], s_tile[4 * j + 1][o], s_tile[4 * j + 2][o], s_tile[4 * j + 3][o]};
      return;
    }
  }
  for (bool first = true; j < n4; j += stride, first = false) {
    if (!first) {
      i = WT ? plain_index(a, j) : j;
      g = reinterpret_cast<const floatx4*>(a.g)[i];
      m = reinterpret_cast<floatx4*>(a.mu)[i];
      v = reinterpret_cast<floatx4*>(a.nu)[i];
      p = reinterpret_cast<floatx4*>(a.p)[i];
    }
    adam_update(a, i, g, m, v, p, norm, clip, bc1, bc2);
  }
}

// Sum of the per-chunk squares in a fixed order: thread t adds chunks
// t, t + 1024, ... in turn, then the block's 1024 partials are added as a
// fixed tree (wave sums, then the 16 wave totals in wave order).
constexpr int NORM_THREADS = 1024;
__global__ void __launch_bounds__(NORM_THREADS) sumsq_total_kernel(const double* __restrict__ sumsq, int n,
                                                                   double* __restrict__ total) {
  __shared__ double w[NORM_THREADS / 64];
  double t = ppo::strided_sum_d<NORM_THREADS, 8>(sumsq, n, threadIdx.x);
  t = ppo::wave_sum_d(t);
  if ((threadIdx.x & 63) == 0) w[threadIdx.x >> 6] = t;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int i = 0; i < NORM_THREADS / 64; ++i) s += w[i];
    total[0] = s;
  }
}

__global__ void count_advance_kernel(int* count_base, int steps, const int* abort_word) {
  if (threadIdx.x == 0 && blockIdx.x == 0 && !(abort_word && *abort_word != 0)) *count_base += steps;
}

}  // namespace

PPO_EXPORT int ppo_grad_reduce_segment_bytes(void) { return (int)sizeof(Segment); }
PPO_EXPORT int ppo_grad_reduce_chunk_bytes(void) { return (int)sizeof(Chunk); }
PPO_EXPORT int ppo_grad_reduce_chunk_elems(void) { return CHUNK; }

// segs/chunks: device tables (layout: ppo_grad_reduce_{segment,chunk}_bytes),
// one block per chunk; sumsq receives nchunks doubles.
// Every segment's count, part stride and pointers must be multiples of 4
// floats (16 bytes): the learner's flat layout guarantees it.
PPO_EXPORT int ppo_grad_reduce(void* stream, const void* segs, const void* chunks, int nchunks, int nfew,
                               int nwide, double* sumsq) {
  if (nchunks < 0 || nfew < 0 || nwide < 0 || nfew + nwide > nchunks || !segs || !chunks || !sumsq)
    return ppo::set_error(PPO_ERR_ARG, "ppo_grad_reduce: bad argument (nchunks=%d nfew=%d nwide=%d)", nchunks,
                          nfew, nwide);
  if (nchunks == 0) return PPO_OK;
  const int blocks = (nfew + 3) / 4 + (nchunks - nfew);
  hipLaunchKernelGGL(grad_reduce_kernel, dim3(blocks), dim3(REDUCE_THREADS), 0, ppo::as_stream(stream),
                     (const Segment*)segs, (const Chunk*)chunks, nchunks, nfew, nwide, sumsq);
  return ppo::check_launch("ppo_grad_reduce");
}

PPO_EXPORT int ppo_grad_reduce_few_parts(void) { return FEW_PARTS; }
PPO_EXPORT int ppo_grad_reduce_wide_parts(void) { return WIDE_PARTS; }
PPO_EXPORT int ppo_grad_reduce_wide_chunk_elems(void) { return WIDE_CHUNK; }

// Hyper-parameters arrive as double, as optax receives Python floats: 1 - b is
// formed in double and rounded once to fp32, like optax's (1 - decay) * g.
PPO_EXPORT int ppo_adam_clip_f32(void* stream, float* params, const float* grads, float* mu, float* nu,
                                 void* params_bf16, int64_t n, const double* sumsq, int nsumsq, double max_norm,
                                 double lr, double b1, double b2, double eps, const int* count_base,
                                 int step_offset, const int* abort_word) {
  if (n < 0 || (n % 4) != 0 || !params || !grads || !mu || !nu || !count_base || (nsumsq > 0 && !sumsq) ||
      nsumsq < 0)
    return ppo::set_error(PPO_ERR_ARG, "ppo_adam_clip_f32: bad argument (n=%lld must be a multiple of 4)",
                          (long long)n);
  if (((uintptr_t)params | (uintptr_t)grads | (uintptr_t)mu | (uintptr_t)nu) & 15u)
    return ppo::set_error(PPO_ERR_ARG, "ppo_adam_clip_f32: buffers must be 16-byte aligned");
  if (n == 0) return PPO_OK;
  AdamParams a{params, grads, mu, nu, params_bf16, n, sumsq, nsumsq, (float)max_norm, (float)(-lr),
               (float)b1, (float)b2, (float)(1.0 - b1), (float)(1.0 - b2), (float)eps, count_base, step_offset,
               abort_word};
  a.ntr = 0;
  a.plain_blocks = (int)std::min<int64_t>(ppo::ceil_div64(n / 4, 256), 2048);
  hipLaunchKernelGGL(adam_kernel<false>, dim3(a.plain_blocks), dim3(256), 0, ppo::as_stream(stream), a);
  return ppo::check_launch("ppo_adam_clip_f32");
}

// ppo_adam_clip_f32 that also writes the transposed image of ntr (at most 8)
// 256 x 256 row-major kernels of the parameters: kernel r starts at element
// tr_off[r] of params (a multiple of 4, the kernels disjoint and inside n),
// and its updated values go to tr_dst[r] as [256 out][256 in] (16-byte
// aligned).  The parameters, moments and bf16 image are the same bits as
// ppo_adam_clip_f32's.
PPO_EXPORT int ppo_adam_clip_wt_f32(void* stream, float* params, const float* grads, float* mu, float* nu,
                                    void* params_bf16, int64_t n, const double* sumsq, int nsumsq, double max_norm,
                                    double lr, double b1, double b2, double eps, const int* count_base,
                                    int step_offset, const int* abort_word, int ntr, const int64_t* tr_off,
                                    float* const* tr_dst) {
  const char* name = "ppo_adam_clip_wt_f32";
  if (n < 0 || (n % 4) != 0 || !params || !grads || !mu || !nu || !count_base || (nsumsq > 0 && !sumsq) ||
      nsumsq < 0 || ntr < 0 || ntr > ADAM_TR_MAX || (ntr > 0 && (!tr_off || !tr_dst)))
    return ppo::set_error(PPO_ERR_ARG, "%s: bad argument (n=%lld, ntr=%d)", name, (long long)n, ntr);
  if (((uintptr_t)params | (uintptr_t)grads | (uintptr_t)mu | (uintptr_t)nu) & 15u)
    return ppo::set_error(PPO_ERR_ARG, "%s: buffers must be 16-byte aligned", name);
  constexpr int64_t KN = 256 * 256;
  for (int r = 0; r < ntr; ++r) {
    if (tr_off[r] < 0 || tr_off[r] % 4 || tr_off[r] + KN > n || !tr_dst[r] || ((uintptr_t)tr_dst[r] & 15u))
      return ppo::set_error(PPO_ERR_ARG, "%s: kernel %d: bad offset %lld or image", name, r, (long long)tr_off[r]);
    for (int q = 0; q < r; ++q)
      if (tr_off[q] < tr_off[r] + KN && tr_off[r] < tr_off[q] + KN)
        return ppo::set_error(PPO_ERR_ARG, "%s: kernels %d and %d overlap", name, q, r);
  }
  if (n == 0) return PPO_OK;
  AdamParams a{params, grads, mu, nu, params_bf16, n, sumsq, nsumsq, (float)max_norm, (float)(-lr),
               (float)b1, (float)b2, (float)(1.0 - b1), (float)(1.0 - b2), (float)eps, count_base, step_offset,
               abort_word};
  // the kernels in ascending offset order (the grid-stride pass skips them in turn)
  int order[ADAM_TR_MAX];
  for (int r = 0; r < ntr; ++r) order[r] = r;
  std::sort(order, order + ntr, [&](int x, int y) { return tr_off[x] < tr_off[y]; });
  a.ntr = ntr;
  for (int r = 0; r < ntr; ++r) {
    a.tr_off[r] = tr_off[order[r]];
    a.tr_dst[r] = tr_dst[order[r]];
  }
  const int64_t plain = n / 4 - (int64_t)ntr * KN / 4;
  a.plain_blocks = (int)std::max<int64_t>(1, std::min<int64_t>(ppo::ceil_div64(plain, 256), 2048));
  a.plain_blocks = (a.plain_blocks + 7) / 8 * 8;
  hipLaunchKernelGGL(adam_kernel<true>, dim3(a.plain_blocks + (256 / TJ_ROWS) * ntr), dim3(256), 0,
                     ppo::as_stream(stream), a);
  return ppo::check_launch(name);
}

// total[0] = sum of sumsq[0..n) in a fixed order (one block): hands the
// optimizer one squared norm instead of every block re-adding n partials.
PPO_EXPORT int ppo_sumsq_total(void* stream, const double* sumsq, int n, double* total) {
  if (n < 0 || !total || (n > 0 && !sumsq)) return ppo::set_error(PPO_ERR_ARG, "ppo_sumsq_total: bad argument");
  hipLaunchKernelGGL(sumsq_total_kernel, dim3(1), dim3(NORM_THREADS), 0, ppo::as_stream(stream), sumsq, n, total);
  return ppo::check_launch("ppo_sumsq_total");
}

PPO_EXPORT int ppo_count_advance(void* stream, int* count_base, int steps, const int* abort_word) {
  if (!count_base) return ppo::set_error(PPO_ERR_ARG, "ppo_count_advance: null counter");
  hipLaunchKernelGGL(count_advance_kernel, dim3(1), dim3(64), 0, ppo::as_stream(stream), count_base, steps,
                     abort_word);
  return ppo::check_launch("ppo_count_advance");
}
