// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), LDS-staged and
// double-buffered, for the Dense layers of the learner's torso:
//
//   forward      Y[M,N]  = act(X[rows(M),K] W[K,N] + b)      (A k-contiguous, B n-contiguous)
//   backward dX  dX[M,K] = (dY[M,N] W[K,N]^T) * act'(aux)    (A k-contiguous, B k-contiguous)
//   backward dW  dW[K,N] = X[rows,K]^T dY[rows,N]             (both operands row-major over the
//                                                             reduction dim; split over rows)
//
// One kernel template covers the three: C[m][n] = sum_k A(m,k) B(k,n) where A is
// stored either [m][k] (A_K) or [k][m], and B either [n][k] (B_K) or [k][n].
// Each operand keeps its global orientation in LDS, so global loads are 16-byte
// vectors along the contiguous axis and no transpose happens on the way in.
//
// Tiling: 256 threads = 4 wave64s in a 2x2 grid; each wave owns a
// (BM/2) x (BN/2) sub-tile made of 32x32 MFMA blocks.  BK = 16 per stage.  The
// reduction index is permuted inside each group of 8 so that lane half h of a
// wave consumes k = 8g + 4h + s at MFMA step s: a k-contiguous operand then
// feeds four MFMAs from one ds_read_b128, the other orientation from four
// conflict-free ds_read_b32 rows.
//
// A row gather (minibatch indices) applies to the rows of X in the forward
// (A_K: row m -> rows[m]) and in dW (reduction row k -> rows[k]), so the
// minibatch is never materialised.  dW also sums B's columns over each split
// for the bias gradient (one extra add per MFMA in the waves of the first row
// tile), and writes one partial per split; partials are reduced in a fixed
// order later, so results do not depend on scheduling.
#include "gemm_f32.h"

#include <algorithm>

namespace {

using namespace ppo_f32;

constexpr int BK_MIN = 16;  // reduction granule: k_per_split is a multiple of it
constexpr int LDS_PAD = 4;

// Four consecutive elements of a (valid) row at i.  Out-of-range elements
// read a clamped valid address and are flagged in `bits` (bit e set: element
// e valid); the zeroing happens when the stage is written to LDS, after the
// MFMAs of the current stage, so the loads stay in flight behind them.
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

template <int BM, int BN, int BK, bool A_K, bool B_K, bool VA, bool VB>
__global__ void __launch_bounds__(256, 2) gemm_f32_kernel(GemmParams p0) {
  constexpr int A_ROWS = A_K ? BM : BK;
  constexpr int A_COLS = A_K ? BK : BM;
  constexpr int B_ROWS = B_K ? BN : BK;
  constexpr int B_COLS = B_K ? BK : BN;
  constexpr int A_PER = (BM * BK / 4) / 256;  // float4 loads per thread per stage
  constexpr int B_PER = (BN * BK / 4) / 256;
  constexpr int MB = BM / 64;  // 32x32 blocks per wave along M
  constexpr int NB = BN / 64;
  static_assert(A_PER >= 1 && B_PER >= 1, "tile too small for 256 threads");

  __shared__ __attribute__((aligned(16))) float sA[2][A_ROWS][A_COLS + LDS_PAD];
  __shared__ __attribute__((aligned(16))) float sB[2][B_ROWS][B_COLS + LDS_PAD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const ppo::TileCoord tc = ppo::xcd_tile();
  const int tower = tc.z / p0.splits;
  const int split = tc.z - tower * p0.splits;
  const GemmParams p = tower_params(p0, tower);
  const int m0 = tc.m * BM;
  const int n0 = tc.n * BN;
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

  floatx4 ra[A_PER], rb[B_PER];
  uint32_t ma[A_PER], mb[B_PER];
  // A_K: each thread's A rows (gathered or not) are the same at every stage
  const float* arow[A_K ? A_PER : 1];
  bool arow_ok[A_K ? A_PER : 1];
  if (A_K) {
#pragma unroll
    for (int j = 0; j < A_PER; ++j) {
      const int gm = m0 + (tid + 256 * j) / (BK / 4);
      const bool ok = gm < p.M;
      const int gmc = ok ? gm : 0;
      const int64_t row = p.rows ? (int64_t)p.rows[gmc] : (int64_t)gmc;
      arow[j] = p.A + row * p.lda;
      arow_ok[j] = ok;
    }
  }

  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < A_PER; ++j) {
      const int f = tid + 256 * j;
      if (A_K) {
        const int c = (f % (BK / 4)) * 4;
        ra[j] = load4<VA>(arow[j], k0 + c, ke, arow_ok[j], ma[j]);
      } else {
        const int r = f / (BM / 4);
        const int c = (f % (BM / 4)) * 4;
        const int k = k0 + r;
        const bool ok = k < ke;
        const int kc = ok ? k : 0;
        const int64_t row = p.rows ? (int64_t)p.rows[kc] : (int64_t)kc;
        ra[j] = load4<VA>(p.A + row * p.lda, m0 + c, p.M, ok, ma[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < B_PER; ++j) {
      const int f = tid + 256 * j;
      if (B_K) {
        const int r = f / (BK / 4);
        const int c = (f % (BK / 4)) * 4;
        const int gn = n0 + r;
        const bool ok = gn < p.N;
        rb[j] = load4<VB>(p.B + (int64_t)(ok ? gn : 0) * p.ldb, k0 + c, ke, ok, mb[j]);
      } else {
        const int r = f / (BN / 4);
        const int c = (f % (BN / 4)) * 4;
        const int k = k0 + r;
        const bool ok = k < ke;
        rb[j] = load4<VB>(p.B + (int64_t)(ok ? k : 0) * p.ldb, n0 + c, p.N, ok, mb[j]);
      }
    }
  };

  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < A_PER; ++j) {
      const int f = tid + 256 * j;
      const int r = A_K ? f / (BK / 4) : f / (BM / 4);
      const int c = A_K ? (f % (BK / 4)) * 4 : (f % (BM / 4)) * 4;
      *reinterpret_cast<floatx4*>(&sA[buf][r][c]) = masked(ra[j], ma[j]);
    }
#pragma unroll
    for (int j = 0; j < B_PER; ++j) {
      const int f = tid + 256 * j;
      const int r = B_K ? f / (BK / 4) : f / (BN / 4);
      const int c = B_K ? (f % (BK / 4)) * 4 : (f % (BN / 4)) * 4;
      *reinterpret_cast<floatx4*>(&sB[buf][r][c]) = masked(rb[j], mb[j]);
    }
  };

  const int nk = (ke > kb) ? (ke - kb + BK - 1) / BK : 0;
  if (nk > 0) {
    gload(kb);
    sstore(0);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kb + (kt + 1) * BK);
#pragma unroll
    for (int g = 0; g < BK / 8; ++g) {
      const int kk = 8 * g + 4 * h;
      floatx4 a4[MB], b4[NB];
#pragma unroll
      for (int bi = 0; bi < MB; ++bi) {
        const int i = wm * (BM / 2) + bi * 32 + l32;
        if (A_K) {
          a4[bi] = *reinterpret_cast<const floatx4*>(&sA[buf][i][kk]);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) a4[bi][s] = sA[buf][kk + s][i];
        }
      }
#pragma unroll
      for (int bj = 0; bj < NB; ++bj) {
        const int j = wn * (BN / 2) + bj * 32 + l32;
        if (B_K) {
          b4[bj] = *reinterpret_cast<const floatx4*>(&sB[buf][j][kk]);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) b4[bj][s] = sB[buf][kk + s][j];
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int bi = 0; bi < MB; ++bi)
#pragma unroll
          for (int bj = 0; bj < NB; ++bj)
            acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[bi][s], b4[bj][s], acc[bi][bj], 0, 0, 0);
      if (do_bsum) {
#pragma unroll
        for (int bj = 0; bj < NB; ++bj) bsum[bj] += (b4[bj][0] + b4[bj][1]) + (b4[bj][2] + b4[bj][3]);
      }
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  float no_aux[MB * NB * 16];
  epilogue_f32<MB, NB>(p, acc, bsum, do_bsum, m0 + wm * (BM / 2), n0 + wn * (BN / 2), split, lane, no_aux);
}

template <int BM, int BN, int BK, bool A_K, bool B_K>
int launch_tile(hipStream_t st, const GemmParams& p, int splits, bool va, bool vb) {
  dim3 grid(ppo::ceil_div(p.N, BN), ppo::ceil_div(p.M, BM), splits * p.towers);
  dim3 block(256);
  if (va && vb) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, A_K, B_K, true, true>), grid, block, 0, st, p);
  else if (va) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, A_K, B_K, true, false>), grid, block, 0, st, p);
  else if (vb) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, A_K, B_K, false, true>), grid, block, 0, st, p);
  else hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, A_K, B_K, false, false>), grid, block, 0, st, p);
  return ppo::check_launch("ppo_gemm_f32");
}

template <bool A_K, bool B_K>
int launch_layout(hipStream_t st, const GemmParams& p, int splits, bool va, bool vb, int tile) {
  switch (tile) {
    case 0: return launch_tile<128, 128, 16, A_K, B_K>(st, p, splits, va, vb);
    case 1: return launch_tile<128, 64, 16, A_K, B_K>(st, p, splits, va, vb);
    case 2: return launch_tile<64, 128, 16, A_K, B_K>(st, p, splits, va, vb);
    case 3: return launch_tile<64, 64, 16, A_K, B_K>(st, p, splits, va, vb);
    case 4: return launch_tile<128, 128, 32, A_K, B_K>(st, p, splits, va, vb);
    case 5: return launch_tile<128, 64, 32, A_K, B_K>(st, p, splits, va, vb);
    case 6: return launch_tile<64, 128, 32, A_K, B_K>(st, p, splits, va, vb);
    case 7: return launch_tile<64, 64, 32, A_K, B_K>(st, p, splits, va, vb);
    default: return launch_tile<128, 128, 16, A_K, B_K>(st, p, splits, va, vb);  // 8, 9 without copies
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// y[r][4 u .. 4 u + 3] = x[r][c] for c < cols, 0 up to ldy: one thread per
// four output columns, one 16-byte store.
__global__ void pad_rows_kernel(const float* __restrict__ x, int64_t ldx, float* __restrict__ y, int64_t ldy,
                                int rows, int cols) {
  const int64_t units = ldy / 4;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)rows * units) return;
  const int64_t r = i / units;
  const int c0 = (int)(i - r * units) * 4;
  const float* xr = x + r * ldx;
  float4 v;
  v.x = c0 < cols ? xr[c0] : 0.f;
  v.y = c0 + 1 < cols ? xr[c0 + 1] : 0.f;
  v.z = c0 + 2 < cols ? xr[c0 + 2] : 0.f;
  v.w = c0 + 3 < cols ? xr[c0 + 3] : 0.f;
  *reinterpret_cast<float4*>(y + r * ldy + c0) = v;
}

}  // namespace

// Generic entry: C[m][n] (+ split * c_split_stride) = epilogue(sum_k A(m,k) B(k,n)).
//   a_layout 0: A[m * lda + k]; 1: A[k * lda + m].   b_layout 0: B[k * ldb + n]; 1: B[n * ldb + k].
//   rows: gather of A's rows (layout 0: over m; layout 1: over k) or null.
//   epi 0: store; 1: bias + activation (pre-activation to `pre` if non-null);
//   2: multiply by act'(aux).  bias_grad (layout a=1, b=0 only): [splits][N] sums of B.
//   tile: -1 picks a tile; 0: 128x128, 1: 128x64, 2: 64x128, 3: 64x64 (copy-fed, 32 reduction
//   elements per stage, when the operands allow; else register-staged with 16); 4-7 the same
//   tiles register-staged with 32 per stage; 8: 128x256 and 9: 256x128 on 8 waves (copy-fed).
static int gemm_f32_impl(void* stream, int a_layout, int b_layout, const float* A, int64_t lda,
                         const int32_t* rows, const float* B, int64_t ldb, float* C, int64_t ldc, int M, int N,
                         int K, int splits, int64_t c_split_stride, int epi, const float* bias, int act, float* pre,
                         const float* aux, int64_t ldaux, float* bias_grad, int tile, int towers,
                         const int64_t* tstride) {
  if (M < 0 || N < 0 || K < 0 || splits < 1 || a_layout < 0 || a_layout > 1 || b_layout < 0 || b_layout > 1 ||
      epi < 0 || epi > 2 || act < 0 || act > 3 || tile > 9 || towers < 1 || towers > 8 ||
      (int64_t)splits * towers > 65535)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_f32: bad argument (M=%d N=%d K=%d splits=%d towers=%d)", M, N, K,
                          splits, towers);
  if (M == 0 || N == 0) return PPO_OK;
  if (!A || !B || !C) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_f32: null operand");
  if (epi == EPI_DACT && !aux) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_f32: EPI_DACT needs aux");
  if (bias_grad && !(a_layout == 1 && b_layout == 0))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_f32: bias_grad needs a_layout=1, b_layout=0");
  if (splits > 1 && c_split_stride < (int64_t)M * ldc)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_f32: split stride too small");
  GemmParams p;
  p.A = A; p.lda = lda; p.rows = rows; p.B = B; p.ldb = ldb; p.C = C; p.ldc = ldc;
  p.c_split_stride = c_split_stride; p.M = M; p.N = N; p.K = K;
  const int kps = ((ppo::ceil_div(K > 0 ? K : 1, splits) + BK_MIN - 1) / BK_MIN) * BK_MIN;
  p.k_per_split = kps;
  p.epi = epi; p.bias = bias; p.act = act; p.pre = pre; p.aux = aux; p.ldaux = ldaux; p.bias_grad = bias_grad;
  p.splits = splits; p.towers = towers;
  p.tA = tstride[0]; p.tB = tstride[1]; p.tC = tstride[2]; p.tBias = tstride[3]; p.tPre = tstride[4];
  p.tAux = tstride[5]; p.tBiasGrad = tstride[6];
  // a tower's strides keep its 16-byte rows aligned
  for (int i = 0; i < 7; ++i)
    if (towers > 1 && tstride[i] % 4 != 0)
      return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_f32_towers: tower strides must be multiples of 4 elements");
  // vector loads need 16-byte rows along the contiguous axis
  const int a_contig = a_layout == 0 ? K : M;
  const int b_contig = b_layout == 1 ? K : N;
  const bool va = (lda % 4 == 0) && (a_contig % 4 == 0) && aligned16(A);
  const bool vb = (ldb % 4 == 0) && (b_contig % 4 == 0) && aligned16(B);
  // Default 64 x 64: three resident workgroups per CU hide latency best over
  // the learner's shapes as a whole inside the update graph (the 8-wave tiles
  // win some isolated launches by 5-10% and lose others by up to 35%).
  if (tile < 0) tile = 3;
  hipStream_t st = ppo::as_stream(stream);
  // Tiles 0-3 and 8-9 run on the copy-fed pipeline (gemm_f32d.hip) whenever
  // every operand row is 16-byte vectorisable and a gathered k-outer A fits
  // its index cache; tiles 4-7 (and the rest) on the register-staged one here
  // (8 and 9 then fall back to 128 x 128).
  const int kps_d = ((ppo::ceil_div(K > 0 ? K : 1, splits) + F32D_BK - 1) / F32D_BK) * F32D_BK;
  const bool dma_tile = tile <= 3 || tile >= 8;
  if (dma_tile && va && vb && !(a_layout == 1 && rows && kps_d > F32D_KIDX_MAX)) {
    p.k_per_split = kps_d;
    return launch_dma(st, p, splits, tile, a_layout, b_layout);
  }
  if (a_layout == 0 && b_layout == 0) return launch_layout<true, false>(st, p, splits, va, vb, tile);
  if (a_layout == 0 && b_layout == 1) return launch_layout<true, true>(st, p, splits, va, vb, tile);
  if (a_layout == 1 && b_layout == 0) return launch_layout<false, false>(st, p, splits, va, vb, tile);
  return launch_layout<false, true>(st, p, splits, va, vb, tile);
}

PPO_EXPORT int ppo_gemm_f32(void* stream, int a_layout, int b_layout, const float* A, int64_t lda,
                            const int32_t* rows, const float* B, int64_t ldb, float* C, int64_t ldc, int M,
                            int N, int K, int splits, int64_t c_split_stride, int epi, const float* bias,
                            int act, float* pre, const float* aux, int64_t ldaux, float* bias_grad, int tile) {
  const int64_t none[7] = {0, 0, 0, 0, 0, 0, 0};
  return gemm_f32_impl(stream, a_layout, b_layout, A, lda, rows, B, ldb, C, ldc, M, N, K, splits, c_split_stride,
                       epi, bias, act, pre, aux, ldaux, bias_grad, tile, 1, none);
}

// ppo_gemm_f32 over `towers` problems of one shape in one grid: problem t's
// A, B, C, bias, pre, aux and bias_grad are the given pointers plus t times
// their stride (elements, multiples of 4; 0 shares the operand, as the
// observation rows both towers of an actor-critic read).
PPO_EXPORT int ppo_gemm_f32_towers(void* stream, int towers, int a_layout, int b_layout, const float* A,
                                   int64_t lda, const int32_t* rows, const float* B, int64_t ldb, float* C,
                                   int64_t ldc, int M, int N, int K, int splits, int64_t c_split_stride, int epi,
                                   const float* bias, int act, float* pre, const float* aux, int64_t ldaux,
                                   float* bias_grad, int tile, int64_t stride_a, int64_t stride_b,
                                   int64_t stride_c, int64_t stride_bias, int64_t stride_pre, int64_t stride_aux,
                                   int64_t stride_bias_grad) {
  const int64_t t[7] = {stride_a, stride_b, stride_c, stride_bias, stride_pre, stride_aux, stride_bias_grad};
  return gemm_f32_impl(stream, a_layout, b_layout, A, lda, rows, B, ldb, C, ldc, M, N, K, splits, c_split_stride,
                       epi, bias, act, pre, aux, ldaux, bias_grad, tile, towers, t);
}

// Row-pitched copy that pads each row with zeros: y[r][c] = x[r][c] for
// c < cols, 0 for cols <= c < ldy (ldy a multiple of 4, y 16-byte aligned; x
// any pitch).  The per-update copy of observation rows whose width is not a
// multiple of four, so that the first layer's weight gradient runs on the
// copy-fed GEMM over the padded width.
PPO_EXPORT int ppo_pad_rows_f32(void* stream, const float* x, int64_t ldx, float* y, int64_t ldy, int rows,
                                int cols) {
  if (rows < 0 || cols < 0 || ldx < cols || ldy < cols || ldy % 4 != 0)
    return ppo::set_error(PPO_ERR_ARG, "ppo_pad_rows_f32: bad shape (rows=%d cols=%d ldx=%lld ldy=%lld)", rows,
                          cols, (long long)ldx, (long long)ldy);
  if (rows == 0 || ldy == 0) return PPO_OK;
  if (!x || !y || !aligned16(y))
    return ppo::set_error(PPO_ERR_ARG, "ppo_pad_rows_f32: buffers must be non-null and y 16-byte aligned");
  const int64_t n = (int64_t)rows * (ldy / 4);
  hipLaunchKernelGGL(pad_rows_kernel, dim3((unsigned)ppo::ceil_div64(n, 256)), dim3(256), 0, ppo::as_stream(stream),
                     x, ldx, y, ldy, rows, cols);
  return ppo::check_launch("ppo_pad_rows_f32");
}

namespace {

// The checked problems of a weight-gradient group (64 x 64 tiles); on error
// the library's error is set and the status returned.  kidx: the largest
// gathered split; all_live: problems with M or N zero are an error instead
// of skipped.
int build_dw_group(const char* name, int count, const float* const* A, const int64_t* lda,
                   const int32_t* const* rows, const float* const* B, const int64_t* ldb, float* const* C,
                   const int64_t* ldc, const int* M, const int* N, const int* K, const int* splits,
                   const int64_t* c_split_stride, float* const* bias_grad, int kidx, bool all_live,
                   ppo_f32::F32Group& g) {
  using namespace ppo_f32;
  if (count < 0 || count > F32_GROUP_MAX || (count > 0 && (!A || !lda || !B || !ldb || !C || !ldc || !M || !N ||
                                                           !K || !splits || !c_split_stride)))
    return ppo::set_error(PPO_ERR_ARG, "%s: bad argument (count=%d, at most %d)", name, count, F32_GROUP_MAX);
  g = F32Group{};
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    if (M[i] < 0 || N[i] < 0 || K[i] < 0 || splits[i] < 1 || splits[i] > 65535 ||
        (all_live && (M[i] == 0 || N[i] == 0)))
      return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: bad shape (M=%d N=%d K=%d splits=%d)", name, i, M[i],
                            N[i], K[i], splits[i]);
    if (M[i] == 0 || N[i] == 0) continue;
    if (!A[i] || !B[i] || !C[i]) return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: null operand", name, i);
    if (splits[i] > 1 && c_split_stride[i] < (int64_t)M[i] * ldc[i])
      return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: split stride too small", name, i);
    if (lda[i] % 4 || M[i] % 4 || lda[i] < M[i] || !aligned16(A[i]) || ldb[i] % 4 || N[i] % 4 || ldb[i] < N[i] ||
        !aligned16(B[i]) || ldc[i] < N[i])
      return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: operand rows must be 16-byte aligned "
                            "with 16-byte vector extents (M=%d N=%d lda=%lld ldb=%lld ldc=%lld)", name, i, M[i], N[i],
                            (long long)lda[i], (long long)ldb[i], (long long)ldc[i]);
    GemmParams& p = g.p[g.count];
    p = GemmParams{};
    p.A = A[i]; p.lda = lda[i]; p.rows = rows ? rows[i] : nullptr; p.B = B[i]; p.ldb = ldb[i];
    p.C = C[i]; p.ldc = ldc[i]; p.c_split_stride = c_split_stride[i]; p.M = M[i]; p.N = N[i]; p.K = K[i];
    p.k_per_split = ((ppo::ceil_div(K[i] > 0 ? K[i] : 1, splits[i]) + F32D_BK - 1) / F32D_BK) * F32D_BK;
    p.epi = EPI_STORE; p.act = 0; p.bias_grad = bias_grad ? bias_grad[i] : nullptr;
    p.splits = splits[i]; p.towers = 1;
    if (p.rows && p.k_per_split > kidx)
      return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: a gathered split holds %d rows (at most %d)", name, i,
                            p.k_per_split, kidx);
    g.gx[g.count] = ppo::ceil_div(N[i], 64);
    g.gy[g.count] = ppo::ceil_div(M[i], 64);
    g.start[g.count] = (int)total;
    total += (int64_t)g.gx[g.count] * g.gy[g.count] * splits[i];
    if (total > (1 << 30)) return ppo::set_error(PPO_ERR_ARG, "%s: too many tiles", name);
    ++g.count;
  }
  g.start[g.count] = (int)total;
  return PPO_OK;
}

}  // namespace

// Weight gradients of several fp32 Dense layers in one launch (64 x 64
// copy-fed tiles): problem i is what ppo_gemm_f32(a_layout = 1, b_layout = 0,
// epi = store, tile = 3) computes from the same arguments, with the same bits.
// Every operand row 16-byte vectorisable (lda, ldb and M[i], N[i] multiples
// of 4, 16-byte aligned pointers); a gathered problem's split holds at most
// F32D_KIDX_MAX rows.
PPO_EXPORT int ppo_gemm_f32_dw_group(void* stream, int count, const float* const* A, const int64_t* lda,
                                     const int32_t* const* rows, const float* const* B, const int64_t* ldb,
                                     float* const* C, const int64_t* ldc, const int* M, const int* N, const int* K,
                                     const int* splits, const int64_t* c_split_stride, float* const* bias_grad) {
  using namespace ppo_f32;
  F32Group g;
  const int rc = build_dw_group("ppo_gemm_f32_dw_group", count, A, lda, rows, B, ldb, C, ldc, M, N, K, splits,
                                c_split_stride, bias_grad, F32D_KIDX_MAX, false, g);
  if (rc != PPO_OK) return rc;
  if (g.start[g.count] == 0) return PPO_OK;
  return launch_dw_group(ppo::as_stream(stream), g);
}

// Output tiles (64 x 64) of a weight-gradient group: the arrival counters and
// squared-norm slots ppo_gemm_f32_dw_group_final uses, problem after problem
// (-1 on a bad shape).
PPO_EXPORT int ppo_gemm_f32_dw_final_slots(int count, const int* M, const int* N) {
  if (count < 0 || count > ppo_f32::F32_GROUP_MAX || (count > 0 && (!M || !N))) return -1;
  int64_t n = 0;
  for (int i = 0; i < count; ++i) {
    if (M[i] <= 0 || N[i] <= 0) return -1;
    n += (int64_t)ppo::ceil_div(M[i], 64) * ppo::ceil_div(N[i], 64);
  }
  return n > (1 << 30) ? -1 : (int)n;
}

// ppo_gemm_f32_dw_group with the gradient assembly of its problems done in
// the same launch: problem i's split partials (C[i], bias_grad[i]) are still
// written, and the last split of each 64 x 64 tile to finish sums them in
// ppo_grad_reduce's fixed order into G[i] (rows < g_rows[i], pitch ldg[i])
// and its bias gradient Gb[i] (or nothing when null), leaving the tile's
// squared-norm partial at sumsq[slot] (slots and counters numbered as
// ppo_gemm_f32_dw_final_slots counts them).  The segments in segs / chunks
// (ppo_grad_reduce's tables, their chunk slots after the tiles') are reduced
// by workgroups of the same launch.  counters: nine zeroed unsigneds per
// tile (one per tile, then eight per tile for the two-level sums of 32 or 64
// splits), left zeroed.  The gradients are the same bits as ppo_gemm_f32_dw_group +
// ppo_grad_reduce over the same segments (the norm partials are grouped by
// tile instead of by chunk).  Splits per problem: 1, 2, 3,
// 4, 6, 8, 12, 16 (one level), 32 or 64 (the last of each group of eight
// splits sums it, the last group the group sums); gathered splits of at most
// F32D_FINAL_KIDX rows.
PPO_EXPORT int ppo_gemm_f32_dw_group_final(void* stream, int count, const float* const* A, const int64_t* lda,
                                           const int32_t* const* rows, const float* const* B, const int64_t* ldb,
                                           float* const* C, const int64_t* ldc, const int* M, const int* N,
                                           const int* K, const int* splits, const int64_t* c_split_stride,
                                           float* const* bias_grad, float* const* G, const int64_t* ldg,
                                           const int* g_rows, float* const* Gb, unsigned* counters, double* sumsq,
                                           const void* segs, const void* chunks, int nchunks, int nfew, int nwide) {
  using namespace ppo_f32;
  const char* name = "ppo_gemm_f32_dw_group_final";
  F32Group g;
  const int rc = build_dw_group(name, count, A, lda, rows, B, ldb, C, ldc, M, N, K, splits, c_split_stride,
                                bias_grad, F32D_FINAL_KIDX, true, g);
  if (rc != PPO_OK) return rc;
  if (count > 0 && (!G || !ldg || !g_rows || !counters || !sumsq))
    return ppo::set_error(PPO_ERR_ARG, "%s: null gradient, counter or norm buffer", name);
  if (nchunks < 0 || nfew < 0 || nwide < 0 || nfew + nwide > nchunks || (nchunks > 0 && (!segs || !chunks)))
    return ppo::set_error(PPO_ERR_ARG, "%s: bad segment tables (nchunks=%d nfew=%d nwide=%d)", name, nchunks, nfew,
                          nwide);
  ppo_gr::DwFinal f = {};
  int slot = 0;
  for (int i = 0; i < count; ++i) {
    const GemmParams& p = g.p[i];
    if (!final_parts_supported(p.splits))
      return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: %d splits (supported: 1, 2, 3, 4, 6, 8, 12, 16, 32, 64)",
                            name, i, p.splits);
    if (!G[i] || !aligned16(G[i]) || ldg[i] % 4 || ldg[i] < p.N || g_rows[i] < 1 || g_rows[i] > p.M)
      return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: bad gradient (g_rows=%d of M=%d, ldg=%lld)", name, i,
                            g_rows[i], p.M, (long long)ldg[i]);
    if (!aligned16(p.C) || p.ldc % 4 || p.c_split_stride % 4 ||
        4 * ((int64_t)p.splits * p.c_split_stride + (int64_t)p.M * p.ldc) > INT32_MAX)
      return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: partials must be 16-byte aligned and under 2 GB", name, i);
    const bool with_bias = Gb && Gb[i] && p.bias_grad;
    if (with_bias && (!aligned16(Gb[i]) || !aligned16(p.bias_grad)))
      return ppo::set_error(PPO_ERR_ARG, "%s: problem %d: bias gradients must be 16-byte aligned", name, i);
    f.G[i] = G[i];
    f.ldg[i] = ldg[i];
    f.g_rows[i] = g_rows[i];
    f.Gb[i] = with_bias ? Gb[i] : nullptr;
    f.slot0[i] = slot;
    f.splits[i] = p.splits;
    slot += g.gx[i] * g.gy[i];
  }
  f.counters = counters;
  f.ntiles = slot;
  f.sumsq = sumsq;
  f.segs = segs;
  f.chunks = chunks;
  f.nchunks = nchunks;
  f.nfew = nfew;
  f.nwide = nwide;
  f.rblocks = nchunks > 0 ? (nfew + 3) / 4 + (nchunks - nfew) : 0;
  f.rpad = (f.rblocks + 7) / 8 * 8;
  if (g.start[g.count] + f.rpad == 0) return PPO_OK;
  return launch_dw_group_final(ppo::as_stream(stream), g, f);
}
