// The whole rollout-side PPO.step (boonta/algorithms/ppo.py:57-74) of a
// shared-trunk MLP actor-critic with a categorical head in one launch: the
// trunk's Dense + activation layers (256 wide, fp32), the shared policy/value
// head and dist.sample_and_log_prob(seed=key) (categorical.h), for the
// discrete Anakin network (400 -> 256 -> 256 ReLU -> 6 logits + value).
//
// A workgroup owns 16 env rows.  Each layer is 16 x 256 outputs on eight
// waves: four column quarters of 64 (v_mfma_f32_16x16x4f32, the column map of
// gemm_ln.hip: lane li of quarter q holds columns 64 q + 4 li .. + 3), each
// quarter's contraction split over two waves by alternate 32-deep k chunks,
// whose partials meet in LDS.  A layer's input is the observation rows (first
// layer, staged in LDS by one burst of loads at the start) or the previous
// layer's activations in LDS; its kernel is read as
// 16-byte rows from global memory (L2: every workgroup reads the same
// kernels).  Two waves per SIMD hide each other's load latency.  The head
// (<= 16 outputs) splits its 256-deep contraction over the eight waves; then
// one 16-lane group per row draws the action from the row's logits in LDS.
// Replaces 3 GEMM launches and the sampling launch per env step.
#include "common.h"
#include "categorical.h"

#include <algorithm>

namespace {

constexpr int SM_THREADS = 512;  // 8 waves: 4 column quarters x 2 k halves
constexpr int SM_ROWS = 16;
constexpr int SM_F = 256;
constexpr int SM_MAX_LAYERS = 4;
constexpr int SM_HEAD = 16;  // head outputs: logits and the value column
constexpr int SM_U = 2;      // 16-deep k steps per chunk
constexpr int SM_CH = 16 * SM_U;  // chunk depth
constexpr int SM_MAX_OBS = 1024;  // observation features staged in LDS
constexpr int SM_XP = SM_MAX_OBS + 4;  // their LDS row pitch
constexpr int SM_STAGE = SM_ROWS * SM_MAX_OBS / 4 / SM_THREADS;  // staged vectors per thread

struct StepMlpArgs {
  const float* obs;
  int64_t ldo;
  int K0;  // observation features
  int L;   // trunk layers
  const float* W[SM_MAX_LAYERS];  // [K_l, 256], rows of 256 floats
  const float* b[SM_MAX_LAYERS];
  int act;
  const float* Wh;
  int64_t ldwh;
  const float* bh;
  int A;  // logits; the value is head column A
  const uint32_t* key;
  float temperature;
  int32_t* action;
  float* log_prob;
  float* value;
  int rows;
};

__device__ __forceinline__ floatx4 mfma4(const float (&a)[4], const float (&b)[4], floatx4 acc) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
  return acc;
}

// acc[j] += A[16 rows, K] W[K, c4 + j] for this lane's four columns, A in
// LDS (row pitch PITCH floats, zero from K up to the next multiple of 64): the
// staged observation rows (first layer) or the previous layer's activations.
// The k range is cut into pairs of SM_CH-deep chunks; the wave of k half
// `khalf` takes chunk `khalf` of every pair (the two k halves of a column
// quarter are two waves).  Double-buffered: the loads of the next chunk are in
// flight while the current chunk's MFMAs run.  Every kernel load is
// unconditional (rows clamped in bounds, values past K zeroed by selects, the
// prefetch past the last chunk repeating it) so that the compiler's wait
// before a chunk's MFMAs leaves the next chunk's loads outstanding.
template <int PITCH>
__device__ __forceinline__ void layer_acc(floatx4 (&acc)[4], const float* as, int K, int khalf, const float* W,
                                          int li, int kq, int c4) {
  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
  auto load = [&](int k0, float (&a)[SM_U][4], floatx4 (&w)[SM_U][4]) {
#pragma unroll
    for (int u = 0; u < SM_U; ++u) {
      const int kb = k0 + 16 * u + 4 * kq;
      const floatx4 x4 = *reinterpret_cast<const floatx4*>(as + li * PITCH + kb);
#pragma unroll
      for (int s = 0; s < 4; ++s) a[u][s] = x4[s];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = kb + s;
        const floatx4 v = *reinterpret_cast<const floatx4*>(W + ((unsigned)min(k, K - 1) * SM_F + (unsigned)c4));
        w[u][s] = k < K ? v : zero;
      }
    }
  };
  auto compute = [&](const float (&a)[SM_U][4], const floatx4 (&w)[SM_U][4]) {
#pragma unroll
    for (int u = 0; u < SM_U; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float bb[4] = {w[u][0][j], w[u][1][j], w[u][2][j], w[u][3][j]};
        acc[j] = mfma4(a[u], bb, acc[j]);
      }
    }
  };
  const int npair = (K + 2 * SM_CH - 1) / (2 * SM_CH);
  auto kof = [&](int i) { return min(i, npair - 1) * 2 * SM_CH + SM_CH * khalf; };
  float a0[SM_U][4], a1[SM_U][4];
  floatx4 w0[SM_U][4], w1[SM_U][4];
  load(kof(0), a0, w0);
  for (int i = 0; i < npair; i += 2) {
    load(kof(i + 1), a1, w1);
    compute(a0, w0);
    if (i + 1 >= npair) break;
    load(kof(i + 2), a0, w0);
    compute(a1, w1);
  }
}

template <bool VA>
__global__ void __launch_bounds__(SM_THREADS) step_mlp_kernel(StepMlpArgs p) {
  __shared__ __attribute__((aligned(16))) float xs[SM_ROWS][SM_XP];
  __shared__ __attribute__((aligned(16))) float h[SM_ROWS][SM_F + 4];
  __shared__ __attribute__((aligned(16))) float red[SM_ROWS][SM_F + 4];
  __shared__ float s_head[8][SM_ROWS][SM_HEAD + 1];
  __shared__ float s_out[SM_ROWS][SM_HEAD + 1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int quarter = wave & 3;  // columns 64 quarter .. + 63
  const int khalf = wave >> 2;   // k chunks SM_CH (2 i + khalf) .. + SM_CH - 1
  const int li = lane & 15;
  const int kq = lane >> 4;
  const int r0 = blockIdx.x * SM_ROWS;
  const int c4 = 64 * quarter + 4 * li;

  // stage the 16 observation rows in LDS, zero past K0 (to a multiple of 64)
  // and for rows past the end: all of the workgroup's loads are issued
  // before the first is waited on
  const int KP = (p.K0 + 63) / 64 * 64;
  if (VA) {
    const int q = KP / 4;  // 16-byte vectors per staged row
    floatx4 xv[SM_STAGE];
#pragma unroll
    for (int j = 0; j < SM_STAGE; ++j) {
      const int v = threadIdx.x + SM_THREADS * j;
      const int rr = min(v / q, SM_ROWS - 1), c = v - (v / q) * q;
      const int r = min(r0 + rr, p.rows - 1);
      const floatx4 x = *reinterpret_cast<const floatx4*>(p.obs + (int64_t)r * p.ldo + min(4 * c, p.K0 - 4));
      xv[j] = (v < SM_ROWS * q && r0 + rr < p.rows && 4 * c < p.K0) ? x : floatx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < SM_STAGE; ++j) {
      const int v = threadIdx.x + SM_THREADS * j;
      if (v < SM_ROWS * q) *reinterpret_cast<floatx4*>(&xs[v / q][4 * (v % q)]) = xv[j];
    }
  } else {
    for (int v = threadIdx.x; v < SM_ROWS * KP; v += SM_THREADS) {
      const int rr = v / KP, c = v - rr * KP;
      xs[rr][c] = (r0 + rr < p.rows && c < p.K0) ? p.obs[(int64_t)(r0 + rr) * p.ldo + c] : 0.f;
    }
  }
  __syncthreads();

  for (int l = 0; l < p.L; ++l) {
    floatx4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (l == 0) {
      layer_acc<SM_XP>(acc, &xs[0][0], p.K0, khalf, p.W[0], li, kq, c4);
    } else {
      layer_acc<SM_F + 4>(acc, &h[0][0], SM_F, khalf, p.W[l], li, kq, c4);
    }
    __syncthreads();  // every wave has read this layer's input from h
    if (khalf == 1) {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        *reinterpret_cast<floatx4*>(&red[4 * kq + v][c4]) = floatx4{acc[0][v], acc[1][v], acc[2][v], acc[3][v]};
    }
    __syncthreads();
    if (khalf == 0) {
      const floatx4 bias4 = p.b[l] ? *reinterpret_cast<const floatx4*>(p.b[l] + c4) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const floatx4 o2 = *reinterpret_cast<const floatx4*>(&red[4 * kq + v][c4]);
        floatx4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = ppo::act_fwd(p.act, (acc[j][v] + o2[j]) + bias4[j]);
        *reinterpret_cast<floatx4*>(&h[4 * kq + v][c4]) = o;
      }
    }
    __syncthreads();
  }

  // head: wave w contracts features 32 w .. 32 w + 31 for all 16 outputs
  {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const bool jv = li < p.ldwh;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kb = 32 * wave + 16 * u + 4 * kq;
      float a[4], bb[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        a[s] = h[li][kb + s];
        const float wv = p.Wh[(int64_t)(kb + s) * p.ldwh + min(li, (int)p.ldwh - 1)];
        bb[s] = jv ? wv : 0.f;
      }
      acc = mfma4(a, bb, acc);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) s_head[wave][4 * kq + v][li] = acc[v];
  }
  __syncthreads();
  // one 16-lane group per row: the first four waves
  const int row = threadIdx.x / 16;
  const int j0 = threadIdx.x % 16;
  if (wave < 4) {
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < 8; w += 2) o += s_head[w][row][j0] + s_head[w + 1][row][j0];
    s_out[row][j0] = o + (j0 < p.ldwh && p.bh ? p.bh[j0] : 0.f);
  }
  __syncthreads();
  if (wave >= 4) return;
  const int r = r0 + row;
  const bool row_ok = r < p.rows;
  int act_i;
  float lp;
  ppo::cat::draw(&s_out[row][0], p.A, row_ok, r, p.key[0], p.key[1], p.temperature, j0, act_i, lp);
  if (row_ok && j0 == 0) {
    p.action[r] = act_i;
    p.log_prob[r] = lp;
    p.value[r] = s_out[row][p.A];
  }
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

PPO_EXPORT int ppo_step_mlp_max_layers() { return SM_MAX_LAYERS; }
PPO_EXPORT int ppo_step_mlp_max_obs() { return SM_MAX_OBS; }

PPO_EXPORT int ppo_step_mlp_categorical_f32(void* stream, const float* obs, int64_t ldo, int rows, int obs_dim,
                                           int layers, const float* const* weights, const int64_t* ldw,
                                           const float* const* biases, int act, const float* head_w,
                                           int64_t ldwh, const float* head_b, int A, const uint32_t* key,
                                           float temperature, int32_t* action, float* log_prob, float* value) {
  if (rows < 0 || obs_dim < 1 || obs_dim > SM_MAX_OBS || ldo < obs_dim || layers < 1 || layers > SM_MAX_LAYERS || act < 0 || act > 3 ||
      A < 1 || A + 1 > ldwh || ldwh > SM_HEAD || !weights || !ldw || !biases)
    return ppo::set_error(PPO_ERR_ARG, "ppo_step_mlp_categorical_f32: bad argument (rows %d obs %d layers %d A %d "
                          "ldwh %lld)", rows, obs_dim, layers, A, (long long)ldwh);
  if (rows == 0) return PPO_OK;
  if (!obs || !head_w || !key || !action || !log_prob || !value)
    return ppo::set_error(PPO_ERR_ARG, "ppo_step_mlp_categorical_f32: null buffer");
  StepMlpArgs a{};
  a.obs = obs; a.ldo = ldo; a.K0 = obs_dim; a.L = layers; a.act = act;
  for (int l = 0; l < layers; ++l) {
    if (!weights[l] || !aligned16(weights[l]) || ldw[l] != SM_F ||
        (biases[l] && !aligned16(biases[l])))
      return ppo::set_error(PPO_ERR_ARG, "ppo_step_mlp_categorical_f32: layer %d needs a 16-byte aligned [K, 256] "
                            "kernel with 256-float rows", l);
    a.W[l] = weights[l]; a.b[l] = biases[l];
  }
  a.Wh = head_w; a.ldwh = ldwh; a.bh = head_b; a.A = A; a.key = key; a.temperature = temperature;
  a.action = action; a.log_prob = log_prob; a.value = value; a.rows = rows;
  const bool va = aligned16(obs) && ldo % 4 == 0 && obs_dim % 4 == 0;
  const dim3 grid(ppo::ceil_div(rows, SM_ROWS)), block(SM_THREADS);
  if (va) {
    hipLaunchKernelGGL(step_mlp_kernel<true>, grid, block, 0, ppo::as_stream(stream), a);
  } else {
    hipLaunchKernelGGL(step_mlp_kernel<false>, grid, block, 0, ppo::as_stream(stream), a);
  }
  return ppo::check_launch("ppo_step_mlp_categorical_f32");
}
