// Dense -> LayerNorm -> activation forward of one torso layer in a single
// launch, for the float32 networks whose LayerNorm layers are 256 wide (the
// Gaussian workload's 4 x 256 towers: flax Dense, LayerNorm, SiLU).
//
//   Z = X W + b             (X rows optionally gathered: row r is X[idx[r]])
//   mean, rstd of each row of Z (fast variance E[z^2] - E[z]^2, as flax)
//   Y = act((Z - mean) rstd gamma + beta)
//
// Z, mean and rstd are kept for the backward, exactly as the separate GEMM
// (EPI_BIAS_ACT) and ppo_layernorm_act_fwd_f32 launches would leave them; Y
// is the next layer's input.  Fusing removes the LayerNorm launch and its
// re-read of Z from the latency-bound chain of small minibatch steps.
//
// Tiling: a workgroup owns 16 rows and all 256 columns, its four waves 64
// columns each as four 16 x 16 blocks on v_mfma_f32_16x16x4f32 (16-deep k
// steps, the loads of four steps issued before their MFMAs; 16-byte loads of
// X rows when they are 16-byte aligned, of W rows always).  Row statistics
// are 16-lane butterflies over each wave's columns, then a sum of the four
// waves' partials through LDS.
#include "common.h"

namespace {

constexpr int GL_THREADS = 256;
constexpr int GL_ROWS = 16;
constexpr int GL_F = 256;  // features: 4 waves x 4 blocks x 16 columns

__device__ __forceinline__ floatx4 mfma4(const float (&a)[4], const float (&b)[4], floatx4 acc) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
  return acc;
}

struct GemmLnArgs {
  const float* X;
  int64_t ldx;
  const int32_t* idx;
  const float* W;
  int64_t ldw;
  const float* bias;
  const float* gamma;
  const float* beta;
  float* Z;
  int64_t ldz;
  float* Y;
  int64_t ldy;
  float* mean;
  float* rstd;
  int M, K;
  float eps;
  int act;
  // tower-batched launches (blockIdx.y = tower): tower t's X, its parameters
  // (W, bias, gamma, beta), its Z / Y rows and its mean / rstd sit t times
  // these strides (elements) after tower 0's
  int64_t tX, tP, tZY, tMR;
};

__device__ __forceinline__ GemmLnArgs tower_args(const GemmLnArgs& a, int t) {
  GemmLnArgs q = a;
  if (t) {
    q.X += t * a.tX;
    q.W += t * a.tP;
    if (q.bias) q.bias += t * a.tP;
    q.gamma += t * a.tP;
    q.beta += t * a.tP;
    q.Z += t * a.tZY;
    q.Y += t * a.tZY;
    q.mean += t * a.tMR;
    q.rstd += t * a.tMR;
  }
  return q;
}

// Column map: block j's MFMA column li of wave w is feature 64 w + 4 li + j,
// so each lane's four columns are adjacent and every W, bias, gamma, beta, Z
// and Y access is one 16-byte vector.
template <bool VA>
__global__ void __launch_bounds__(GL_THREADS) gemm_ln_fwd_kernel(GemmLnArgs p0) {
  const GemmLnArgs p = tower_args(p0, blockIdx.y);
  __shared__ float s_sum[4][GL_ROWS];
  __shared__ float s_sq[4][GL_ROWS];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;  // A row; B / D column within a block
  const int kq = lane >> 4;  // k group; D rows 4 kq + v
  const int r0 = blockIdx.x * GL_ROWS;
  const int ra = r0 + li;  // the A row this lane loads
  const bool a_live = ra < p.M;
  const float* xrow = p.X + (a_live ? (int64_t)(p.idx ? p.idx[ra] : ra) * p.ldx : 0);
  const int c4 = 64 * wave + 4 * li;  // this lane's four adjacent columns (blocks j = 0..3)

  floatx4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // 64-deep k chunks, double-buffered: the loads of chunk c + 1 are in flight
  // while chunk c's MFMAs run
  auto load = [&](int k0, float (&a)[4][4], floatx4 (&w)[4][4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int kb = k0 + 16 * u + 4 * kq;
      if (VA) {
        const floatx4 x4 = (a_live && kb < p.K) ? *reinterpret_cast<const floatx4*>(xrow + kb)
                                                  : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) a[u][s] = x4[s];
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) a[u][s] = (a_live && kb + s < p.K) ? xrow[kb + s] : 0.f;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = kb + s;
        w[u][s] = k < p.K ? *reinterpret_cast<const floatx4*>(p.W + (int64_t)k * p.ldw + c4)
                          : floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  auto compute = [&](const float (&a)[4][4], const floatx4 (&w)[4][4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float b[4] = {w[u][0][j], w[u][1][j], w[u][2][j], w[u][3][j]};
        acc[j] = mfma4(a[u], b, acc[j]);
      }
    }
  };
  float a0[4][4], a1[4][4];
  floatx4 w0[4][4], w1[4][4];
  load(0, a0, w0);
  for (int k0 = 0; k0 < p.K; k0 += 128) {
    if (k0 + 64 < p.K) load(k0 + 64, a1, w1);
    compute(a0, w0);
    if (k0 + 64 >= p.K) break;
    if (k0 + 128 < p.K) load(k0 + 128, a0, w0);
    compute(a1, w1);
  }

  // Z = acc + bias; per-row partial sums over this wave's 64 columns
  const floatx4 bias4 = p.bias ? *reinterpret_cast<const floatx4*>(p.bias + c4) : floatx4{0.f, 0.f, 0.f, 0.f};
  float z[4][4];  // [row v][column j]
  float ps[4], pq[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    ps[v] = 0.f;
    pq[v] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      z[v][j] = acc[j][v] + bias4[j];
      ppo::ln_accum(z[v][j], ps[v], pq[v]);
    }
    ps[v] = ppo::sum16(ps[v]);
    pq[v] = ppo::sum16(pq[v]);
  }
  if (li == 0) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      s_sum[wave][4 * kq + v] = ps[v];
      s_sq[wave][4 * kq + v] = pq[v];
    }
  }
  __syncthreads();
  const floatx4 g4 = *reinterpret_cast<const floatx4*>(p.gamma + c4);
  const floatx4 be4 = *reinterpret_cast<const floatx4*>(p.beta + c4);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int rr = 4 * kq + v;
    const int row = r0 + rr;
    const float s = (s_sum[0][rr] + s_sum[1][rr]) + (s_sum[2][rr] + s_sum[3][rr]);
    const float s2 = (s_sq[0][rr] + s_sq[1][rr]) + (s_sq[2][rr] + s_sq[3][rr]);
    float mean, rstd;
    ppo::ln_stats256(s, s2, p.eps, mean, rstd);
    if (row >= p.M) continue;
    if (wave == 0 && li == 0) {
      p.mean[row] = mean;
      p.rstd[row] = rstd;
    }
    floatx4 zo, yo;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      zo[j] = z[v][j];
      yo[j] = ppo::act_fwd(p.act, ppo::ln_apply(z[v][j], mean, rstd, g4[j], be4[j]));
    }
    *reinterpret_cast<floatx4*>(p.Z + (int64_t)row * p.ldz + c4) = zo;
    *reinterpret_cast<floatx4*>(p.Y + (int64_t)row * p.ldy + c4) = yo;
  }
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

static int gemm_ln_impl(void* stream, const float* X, int64_t ldx, const int32_t* rows_idx, const float* W,
                        int64_t ldw, const float* bias, const float* gamma, const float* beta, float* Z, int64_t ldz,
                        float* Y, int64_t ldy, float* mean, float* rstd, int M, int K, int F, float eps, int act,
                        int towers, int64_t tX, int64_t tP, int64_t tZY, int64_t tMR) {
  if (M < 0 || K < 1 || F != GL_F || act < 0 || act > 3 || ldx < K || ldw < F || ldz < F || ldy < F ||
      towers < 1 || towers > 8 || (towers > 1 && (tX % 4 || tP % 4 || tZY % 4)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_ln_act_fwd_f32: bad argument (M=%d K=%d F=%d, F must be %d)", M, K,
                          F, GL_F);
  if (M == 0) return PPO_OK;
  if (!X || !W || !gamma || !beta || !Z || !Y || !mean || !rstd)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_ln_act_fwd_f32: null buffer");
  // W, bias, gamma, beta, Z and Y are read / written as 16-byte vectors
  if (!aligned16(W) || ldw % 4 || (bias && !aligned16(bias)) || !aligned16(gamma) || !aligned16(beta) ||
      !aligned16(Z) || ldz % 4 || !aligned16(Y) || ldy % 4)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_ln_act_fwd_f32: W, bias, gamma, beta, Z, Y need 16-byte rows");
  GemmLnArgs a{X, ldx, rows_idx, W, ldw, bias, gamma, beta, Z, ldz, Y, ldy, mean, rstd, M, K, eps, act,
               tX, tP, tZY, tMR};
  const bool va = aligned16(X) && ldx % 4 == 0 && K % 4 == 0;
  const dim3 grid(ppo::ceil_div(M, GL_ROWS), towers), block(GL_THREADS);
  if (va) {
    hipLaunchKernelGGL(gemm_ln_fwd_kernel<true>, grid, block, 0, ppo::as_stream(stream), a);
  } else {
    hipLaunchKernelGGL(gemm_ln_fwd_kernel<false>, grid, block, 0, ppo::as_stream(stream), a);
  }
  return ppo::check_launch("ppo_gemm_ln_act_fwd_f32");
}

PPO_EXPORT int ppo_gemm_ln_act_fwd_f32(void* stream, const float* X, int64_t ldx, const int32_t* rows_idx,
                                      const float* W, int64_t ldw, const float* bias, const float* gamma,
                                      const float* beta, float* Z, int64_t ldz, float* Y, int64_t ldy, float* mean,
                                      float* rstd, int M, int K, int F, float eps, int act) {
  return gemm_ln_impl(stream, X, ldx, rows_idx, W, ldw, bias, gamma, beta, Z, ldz, Y, ldy, mean, rstd, M, K, F, eps,
                      act, 1, 0, 0, 0, 0);
}

// ppo_gemm_ln_act_fwd_f32 over `towers` layers of one shape in one grid:
// tower t reads X + t stride_x (0: both towers read the same rows), its
// parameters at + t stride_params, and writes Z / Y at + t stride_rows and
// mean / rstd at + t stride_stats (elements; all but the last multiples of 4).
PPO_EXPORT int ppo_gemm_ln_act_fwd_f32_towers(void* stream, int towers, const float* X, int64_t ldx,
                                             const int32_t* rows_idx, const float* W, int64_t ldw, const float* bias,
                                             const float* gamma, const float* beta, float* Z, int64_t ldz, float* Y,
                                             int64_t ldy, float* mean, float* rstd, int M, int K, int F, float eps,
                                             int act, int64_t stride_x, int64_t stride_params, int64_t stride_rows,
                                             int64_t stride_stats) {
  return gemm_ln_impl(stream, X, ldx, rows_idx, W, ldw, bias, gamma, beta, Z, ldz, Y, ldy, mean, rstd, M, K, F, eps,
                      act, towers, stride_x, stride_params, stride_rows, stride_stats);
}
