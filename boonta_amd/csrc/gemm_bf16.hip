// bf16 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x16_bf16, fp32 accumulate)
// for the Dense layers of a bf16-compute network (flax Dense with
// dtype=bfloat16, param_dtype=float32, as boonta's mixed precision composes
// them: boonta/networks/README.md:73-77).
//
// Flax casts the input, kernel and bias of such a layer to bf16, the dot
// accumulates in fp32 and returns bf16, and the bias add runs in bf16; under
// jax.value_and_grad every cotangent of a bf16 value is bf16 and the
// kernel's gradient is a bf16 dot converted back to fp32.  This kernel keeps
// every operand in fp32 storage and rounds to bf16 (round to nearest even)
// exactly where those casts happen:
//   - both operands are rounded to bf16 as they are staged into LDS (the cast
//     of the input, of the fp32 parameters and of an fp32 cotangent);
//   - the epilogue can round the fp32 accumulator to bf16 (the dot's bf16
//     result), add the bf16-rounded bias and round again, then apply the
//     activation (and round once more), storing the bf16 value in fp32;
//   - dW partials stay fp32; the gradient assembly rounds their sum.
//
// Tiling: 256 threads = 4 wave64s in a 2x2 grid, each wave a (BM/2) x (BN/2)
// sub-tile of 32x32 blocks; BK = 32 per stage, LDS double buffer.  Both
// operands sit in LDS k-contiguous ([row][k], bf16), so each lane's MFMA
// operand (8 consecutive k of one row) is one 16-byte LDS read.  An operand
// stored k-contiguous in memory is copied straight (8 k per 16-byte store);
// one stored with the other orientation is transposed on the way in, two k
// rows at a time so every LDS store is a packed bf16 pair.  The minibatch row
// gather applies as in the fp32 GEMM (rows of X in the forward, reduction
// rows in dW).
#include "common.h"

#include <algorithm>

namespace {

constexpr int BK = 32;
constexpr int KPAD = 8;  // bf16 elements of row padding in LDS

enum Epilogue { EPI_STORE = 0, EPI_BIAS_ACT = 1, EPI_DACT = 2 };

struct GemmParams {
  const float* A;
  int64_t lda;
  const int32_t* rows;
  const float* B;
  int64_t ldb;
  float* C;
  int64_t ldc;
  int64_t c_split_stride;
  int M, N, K;
  int k_per_split;
  int epi;
  const float* bias;
  int act;
  int round_out;
  const float* aux;
  int64_t ldaux;
  float* bias_grad;
};

using ppo::bf16_bits;
using ppo::bf16_round;

__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return bf16_bits(lo) | (bf16_bits(hi) << 16); }

// Four consecutive elements of a (valid) row at i; out-of-range elements read a
// clamped valid address and are flagged in `bits` (bit e set: element e valid).
// They are zeroed when the stage is written to LDS, after the current stage's
// MFMAs, so the loads stay in flight behind them.
template <bool VEC>
__device__ __forceinline__ floatx4 load4(const float* __restrict__ p, int i, int lim, bool ok, uint32_t& bits) {
  floatx4 v;
  if (VEC) {
    const bool in = ok && i < lim;
    v = *reinterpret_cast<const floatx4*>(p + (in ? i : 0));
    bits = in ? 0xfu : 0u;
  } else {
    bits = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = ok && i + e < lim;
      v[e] = p[in ? i + e : 0];
      bits |= in ? (1u << e) : 0u;
    }
  }
  return v;
}

__device__ __forceinline__ floatx4 masked(floatx4 v, uint32_t bits) {
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = ((bits >> e) & 1u) ? v[e] : 0.f;
  return v;
}

// One operand's stage: ROWS (m or n) x BK, from memory that is either
// k-contiguous (KC: [row][k]) or row-contiguous ([k][row]).
template <int ROWS, bool KC, bool V>
struct Stage {
  static constexpr int UNITS = ROWS * BK / 8;  // 8 elements per unit
  static constexpr int PER = UNITS / 256;
  static_assert(PER >= 1 && UNITS % 256 == 0, "tile too small for 256 threads");
  floatx4 r[PER][2];
  uint32_t bits[PER][2];
  const float* rowp[KC ? PER : 1];  // KC: this thread's rows, fixed for every stage
  bool row_ok[KC ? PER : 1];

  // KC only: resolve (and gather) the thread's rows once.
  __device__ __forceinline__ void init(const float* __restrict__ base, int64_t ld, int r0, int lim_row,
                                       const int32_t* rows_idx, int tid) {
    if (!KC) return;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int g = r0 + (tid + 256 * j) / (BK / 8);
      const bool ok = g < lim_row;
      const int gc = ok ? g : 0;
      const int64_t row = rows_idx ? (int64_t)rows_idx[gc] : (int64_t)gc;
      rowp[j] = base + row * ld;
      row_ok[j] = ok;
    }
  }

  // k0, ke: k range of this stage and of the split; !KC: base/ld/r0/lim_row
  // address [k][row] memory and rows_idx gathers over k.
  __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int r0, int lim_row, int k0,
                                       int ke, const int32_t* rows_idx, int tid) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int f = tid + 256 * j;
      if (KC) {
        const int c = (f % (BK / 8)) * 8;
        r[j][0] = load4<V>(rowp[j], k0 + c, ke, row_ok[j], bits[j][0]);
        r[j][1] = load4<V>(rowp[j], k0 + c + 4, ke, row_ok[j], bits[j][1]);
      } else {
        const int kp = f / (ROWS / 4);        // k pair within the stage
        const int c = (f % (ROWS / 4)) * 4;   // 4 consecutive rows
        const int k = k0 + 2 * kp;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const bool ok = k + q < ke;
          const int kc = ok ? k + q : 0;
          const int64_t row = rows_idx ? (int64_t)rows_idx[kc] : (int64_t)kc;
          r[j][q] = load4<V>(base + row * ld, r0 + c, lim_row, ok, bits[j][q]);
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t (*s)[BK + KPAD], int tid) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int f = tid + 256 * j;
      const floatx4 a = masked(r[j][0], bits[j][0]);
      const floatx4 b = masked(r[j][1], bits[j][1]);
      if (KC) {
        const int rr = f / (BK / 8);
        const int c = (f % (BK / 8)) * 8;
        uint4 v;
        v.x = pack2(a[0], a[1]);
        v.y = pack2(a[2], a[3]);
        v.z = pack2(b[0], b[1]);
        v.w = pack2(b[2], b[3]);
        *reinterpret_cast<uint4*>(&s[rr][c]) = v;
      } else {
        const int kp = f / (ROWS / 4);
        const int c = (f % (ROWS / 4)) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          *reinterpret_cast<uint32_t*>(&s[c + e][2 * kp]) = pack2(a[e], b[e]);
      }
    }
  }
};

__device__ __forceinline__ float act_apply(int act, float v, bool round) {
  if (act == ACT_NONE) return v;
  const float y = ppo::act_fwd(act, v);
  return round ? bf16_round(y) : y;
}

// The wave's MB x NB blocks of 32 x 32 from row wm0, column wn0 through the
// epilogue; EPI_ / ACT_: the epilogue kind and activation as compile-time
// constants (the unrolled element loop then holds only their code), -1 for
// the run-time values.
template <int EPI_, int ACT_, int MB, int NB>
__device__ __forceinline__ void epilogue_bf16(const GemmParams& p, float* C, floatx16 (&acc)[MB][NB], int wm0, int wn0,
                                              int h, int l32) {
  const int epi = EPI_ >= 0 ? EPI_ : p.epi;
  const int act = ACT_ >= 0 ? ACT_ : p.act;
  const bool rnd = p.round_out != 0;
#pragma unroll
  for (int bi = 0; bi < MB; ++bi) {
#pragma unroll
    for (int bj = 0; bj < NB; ++bj) {
      const int gn = wn0 + bj * 32 + l32;
      const bool n_ok = gn < p.N;
      float bias = 0.f;
      if (epi == EPI_BIAS_ACT && p.bias && n_ok) bias = rnd ? bf16_round(p.bias[gn]) : p.bias[gn];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = wm0 + bi * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (!n_ok || gm >= p.M) continue;
        float v = acc[bi][bj][r];
        if (rnd) v = bf16_round(v);
        const int64_t o = (int64_t)gm * p.ldc + gn;
        if (epi == EPI_BIAS_ACT) {
          if (p.bias) {
            v += bias;
            if (rnd) v = bf16_round(v);
          }
          v = act_apply(act, v, rnd);
        } else if (epi == EPI_DACT) {
          v *= ppo::act_grad(act, p.aux[(int64_t)gm * p.ldaux + gn]);
          if (rnd) v = bf16_round(v);
        }
        C[o] = v;
      }
    }
  }
}

template <int BM, int BN, bool A_K, bool B_K, bool VA, bool VB>
__global__ void __launch_bounds__(256, 2) gemm_bf16_kernel(GemmParams p) {
  constexpr int MB = BM / 64;
  constexpr int NB = BN / 64;
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM][BK + KPAD];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN][BK + KPAD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const ppo::TileCoord tc = ppo::xcd_tile();
  const int m0 = tc.m * BM;
  const int n0 = tc.n * BN;
  const int split = tc.z;
  const int kb = split * p.k_per_split;
  const int ke = min(p.K, kb + p.k_per_split);

  floatx16 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float bsum[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) bsum[j] = 0.f;
  const bool do_bsum = (p.bias_grad != nullptr) && (tc.m == 0) && (wm == 0);

  Stage<BM, A_K, VA> sa;
  Stage<BN, B_K, VB> sb;
  sa.init(p.A, p.lda, m0, p.M, p.rows, tid);
  sb.init(p.B, p.ldb, n0, p.N, nullptr, tid);
  // A rows are m (A_K) or the gathered reduction rows (!A_K); B never gathers.
  auto gload = [&](int k0) {
    sa.load(p.A, p.lda, m0, p.M, k0, ke, p.rows, tid);
    sb.load(p.B, p.ldb, n0, p.N, k0, ke, nullptr, tid);
  };

  const int nk = (ke > kb) ? (ke - kb + BK - 1) / BK : 0;
  if (nk > 0) {
    gload(kb);
    sa.store(sA[0], tid);
    sb.store(sB[0], tid);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kb + (kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 a8[MB], b8[NB];
#pragma unroll
      for (int bi = 0; bi < MB; ++bi)
        a8[bi] = *reinterpret_cast<const bf16x8*>(&sA[buf][wm * (BM / 2) + bi * 32 + l32][kk + 8 * h]);
#pragma unroll
      for (int bj = 0; bj < NB; ++bj)
        b8[bj] = *reinterpret_cast<const bf16x8*>(&sB[buf][wn * (BN / 2) + bj * 32 + l32][kk + 8 * h]);
#pragma unroll
      for (int bi = 0; bi < MB; ++bi)
#pragma unroll
        for (int bj = 0; bj < NB; ++bj)
          acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8[bi], b8[bj], acc[bi][bj], 0, 0, 0);
      if (do_bsum) {
#pragma unroll
        for (int bj = 0; bj < NB; ++bj) {
          float t = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) t += (float)b8[bj][e];
          bsum[bj] += t;
        }
      }
    }
    if (kt + 1 < nk) {
      sa.store(sA[buf ^ 1], tid);
      sb.store(sB[buf ^ 1], tid);
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
  // (the workloads' forms as compile-time constants; others at run time)
  float* C = p.C + (int64_t)split * p.c_split_stride;
  const int wm0 = m0 + wm * (BM / 2), wn0 = n0 + wn * (BN / 2);
  if (p.epi == EPI_STORE)
    epilogue_bf16<EPI_STORE, ACT_NONE, MB, NB>(p, C, acc, wm0, wn0, h, l32);
  else if (p.epi == EPI_BIAS_ACT && p.act == ACT_NONE)
    epilogue_bf16<EPI_BIAS_ACT, ACT_NONE, MB, NB>(p, C, acc, wm0, wn0, h, l32);
  else if (p.epi == EPI_DACT && p.act == ACT_RELU)
    epilogue_bf16<EPI_DACT, ACT_RELU, MB, NB>(p, C, acc, wm0, wn0, h, l32);
  else
    epilogue_bf16<-1, -1, MB, NB>(p, C, acc, wm0, wn0, h, l32);
  if (do_bsum) {
#pragma unroll
    for (int bj = 0; bj < NB; ++bj) {
      const float t = ppo::add_xor32(bsum[bj]);
      const int gn = n0 + wn * (BN / 2) + bj * 32 + l32;
      if (h == 0 && gn < p.N) p.bias_grad[(int64_t)split * p.N + gn] = t;
    }
  }
}

template <int BM, int BN, bool A_K, bool B_K>
int launch_tile(hipStream_t st, const GemmParams& p, int splits, bool va, bool vb) {
  dim3 grid(ppo::ceil_div(p.N, BN), ppo::ceil_div(p.M, BM), splits);
  dim3 block(256);
  if (va && vb) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, A_K, B_K, true, true>), grid, block, 0, st, p);
  else if (va) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, A_K, B_K, true, false>), grid, block, 0, st, p);
  else if (vb) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, A_K, B_K, false, true>), grid, block, 0, st, p);
  else hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, A_K, B_K, false, false>), grid, block, 0, st, p);
  return ppo::check_launch("ppo_gemm_bf16");
}

template <bool A_K, bool B_K>
int launch_layout(hipStream_t st, const GemmParams& p, int splits, bool va, bool vb, int tile) {
  switch (tile) {
    case 0: return launch_tile<128, 128, A_K, B_K>(st, p, splits, va, vb);
    case 1: return launch_tile<128, 64, A_K, B_K>(st, p, splits, va, vb);
    case 2: return launch_tile<64, 128, A_K, B_K>(st, p, splits, va, vb);
    default: return launch_tile<64, 64, A_K, B_K>(st, p, splits, va, vb);
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

// C[m][n] (+ split * c_split_stride) = epilogue(sum_k bf16(A(m,k)) bf16(B(k,n))), fp32 accumulate.
// Layouts, gather, splits and bias_grad as ppo_gemm_f32.  round_out: round the
// result to bf16 (and, with epi 1, round the bias, the biased value and the
// activation output), as flax does for a bf16 Dense.
PPO_EXPORT int ppo_gemm_bf16(void* stream, int a_layout, int b_layout, const float* A, int64_t lda,
                             const int32_t* rows, const float* B, int64_t ldb, float* C, int64_t ldc, int M,
                             int N, int K, int splits, int64_t c_split_stride, int epi, const float* bias,
                             int act, int round_out, const float* aux, int64_t ldaux, float* bias_grad, int tile) {
  if (M < 0 || N < 0 || K < 0 || splits < 1 || a_layout < 0 || a_layout > 1 || b_layout < 0 || b_layout > 1 ||
      epi < 0 || epi > 2 || act < 0 || act > 3)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16: bad argument (M=%d N=%d K=%d splits=%d)", M, N, K, splits);
  if (M == 0 || N == 0) return PPO_OK;
  if (!A || !B || !C) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16: null operand");
  if (epi == EPI_DACT && !aux) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16: EPI_DACT needs aux");
  if (bias_grad && !(a_layout == 1 && b_layout == 0))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16: bias_grad needs a_layout=1, b_layout=0");
  if (splits > 1 && c_split_stride < (int64_t)M * ldc)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16: split stride too small");
  GemmParams p;
  p.A = A; p.lda = lda; p.rows = rows; p.B = B; p.ldb = ldb; p.C = C; p.ldc = ldc;
  p.c_split_stride = c_split_stride; p.M = M; p.N = N; p.K = K;
  p.k_per_split = ((ppo::ceil_div(K > 0 ? K : 1, splits) + BK - 1) / BK) * BK;
  p.epi = epi; p.bias = bias; p.act = act; p.round_out = round_out; p.aux = aux; p.ldaux = ldaux;
  p.bias_grad = bias_grad;
  const int a_contig = a_layout == 0 ? K : M;
  const int b_contig = b_layout == 1 ? K : N;
  const bool va = (lda % 4 == 0) && (a_contig % 4 == 0) && aligned16(A);
  const bool vb = (ldb % 4 == 0) && (b_contig % 4 == 0) && aligned16(B);
  // 64 x 128 for long reductions (the first layer's 8268 features), 64 x 64
  // otherwise: the measured best on the learner shapes.
  if (tile < 0) tile = (K >= 2048 && (int64_t)ppo::ceil_div(M, 64) * ppo::ceil_div(N, 128) * splits >= 256) ? 2 : 3;
  hipStream_t st = ppo::as_stream(stream);
  if (a_layout == 0 && b_layout == 0) return launch_layout<true, false>(st, p, splits, va, vb, tile);
  if (a_layout == 0 && b_layout == 1) return launch_layout<true, true>(st, p, splits, va, vb, tile);
  if (a_layout == 1 && b_layout == 0) return launch_layout<false, false>(st, p, splits, va, vb, tile);
  return launch_layout<false, true>(st, p, splits, va, vb, tile);
}

// In-place rounding of n fp32 values to bf16 (round to nearest even).
namespace {
__global__ void round_bf16_kernel(float* x, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    x[i] = bf16_round(x[i]);
}
}  // namespace

PPO_EXPORT int ppo_round_bf16(void* stream, float* x, int64_t n) {
  if (n < 0) return ppo::set_error(PPO_ERR_ARG, "ppo_round_bf16: negative size");
  if (n == 0) return PPO_OK;
  if (!x) return ppo::set_error(PPO_ERR_ARG, "ppo_round_bf16: null buffer");
  const int64_t blocks = std::min<int64_t>(ppo::ceil_div64(n, 256), 4096);
  hipLaunchKernelGGL(round_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, ppo::as_stream(stream), x, n);
  return ppo::check_launch("ppo_round_bf16");
}
