// bf16 GEMM for the long reductions of a bf16-compute network: the first
// layer of the large-observation network (8192 gathered rows x 8268 features
// -> 512, forward and dW), where operands stream from HBM.
//
// Same contraction, layouts, row gather, split-K, epilogues and flax rounding
// points as ppo_gemm_bf16 (see gemm_bf16.hip), with operands that may be
// stored as bf16 (the observation copy and the bf16 image of the parameters)
// or fp32 (rounded to bf16 as they are staged).  What differs is the
// pipeline, sized for bf16 MFMA rates:
//   - 256 x 128 output tile, 8 wave64s (4 x 2, each 64 x 64 = 2 x 2 blocks of
//     v_mfma_f32_32x32x16_bf16), BK = 64 per stage;
//   - two register sets of staged loads, so the loads of stage k + 2 are in
//     flight while stage k is multiplied and stage k + 1 is written to LDS
//     (two stages of MFMA work cover a global-load round trip);
//   - operands sit in LDS k-contiguous ([row][k], bf16, 16-byte rows), so an
//     MFMA operand (8 consecutive k of one row) is one 16-byte LDS read; an
//     operand stored with the other orientation is transposed on the way in,
//     two k rows at a time so every LDS store is a packed bf16 pair.
#include "common.h"

#include <algorithm>

namespace {

constexpr int BK = 64;
constexpr int KPAD = 8;
constexpr int LDK = BK + KPAD;  // LDS row pitch (bf16 elements)

enum Epilogue { EPI_STORE = 0, EPI_BIAS_ACT = 1, EPI_DACT = 2 };

struct Params {
  const void* A;
  int64_t lda;
  const int32_t* rows;
  const void* B;
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

// Raw staged data of one unit (8 consecutive elements along the contiguous
// axis) and its validity, converted and masked only when written to LDS, so
// a stage's loads stay in flight behind the current stage's MFMAs.
template <typename T>
struct Unit;

template <>
struct Unit<float> {
  floatx4 a, b;
  uint32_t bits;  // bit e: element e valid
  __device__ __forceinline__ void load(const float* __restrict__ p, int i, int lim, bool ok) {
    bits = 0u;
    const bool in0 = ok && i < lim, in1 = ok && i + 4 < lim;  // fp32 extents are multiples of 4
    a = *reinterpret_cast<const floatx4*>(p + (in0 ? i : 0));
    b = *reinterpret_cast<const floatx4*>(p + (in1 ? i + 4 : 0));
    bits = (in0 ? 0x0fu : 0u) | (in1 ? 0xf0u : 0u);
  }
  __device__ __forceinline__ uint4 packed() const {
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = ((bits >> e) & 1u) ? a[e] : 0.f;
      x[e + 4] = ((bits >> (e + 4)) & 1u) ? b[e] : 0.f;
    }
    uint4 v;
    v.x = pack2(x[0], x[1]);
    v.y = pack2(x[2], x[3]);
    v.z = pack2(x[4], x[5]);
    v.w = pack2(x[6], x[7]);
    return v;
  }
};

// bf16 rows: a 16-byte load may run past `lim` into the row's padding (the
// leading dimension is at least lim rounded up to 8); those elements are zeroed.
template <>
struct Unit<uint16_t> {
  uint4 v;
  int valid;  // elements valid from the start (0..8)
  __device__ __forceinline__ void load(const uint16_t* __restrict__ p, int i, int lim, bool ok) {
    const bool in = ok && i < lim;
    v = *reinterpret_cast<const uint4*>(p + (in ? i : 0));
    valid = in ? min(8, lim - i) : 0;
  }
  __device__ __forceinline__ uint4 packed() const {
    uint4 out = v;
    uint32_t* w = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] &= (2 * e + 1 < valid) ? 0xffffffffu : (2 * e < valid ? 0x0000ffffu : 0u);
    return out;
  }
};

// One operand's stage: ROWS (m or n) x BK, NT threads.  KC: memory is
// [row][k] (k contiguous); otherwise [k][row].  A !KC unit pairs two k rows.
template <int ROWS, bool KC, typename T, int NT>
struct Stage {
  static constexpr int UNITS = KC ? ROWS * BK / 8 : ROWS * BK / 16;
  static constexpr int PER = UNITS / NT;
  static_assert(PER >= 1 && UNITS % NT == 0, "tile too small for the thread count");
  Unit<T> u[PER][KC ? 1 : 2];
};

// KC rows of one thread, resolved (and gathered) once for every stage.
template <int ROWS, bool KC, typename T, int NT>
struct Rows {
  static constexpr int PER = Stage<ROWS, KC, T, NT>::PER;
  const T* p[KC ? PER : 1];
  bool ok[KC ? PER : 1];
  __device__ __forceinline__ void init(const T* base, int64_t ld, int r0, int lim_row, const int32_t* rows_idx,
                                       int tid) {
    if (!KC) return;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int g = r0 + (tid + NT * j) / (BK / 8);
      const bool in = g < lim_row;
      const int gc = in ? g : 0;
      const int64_t row = rows_idx ? (int64_t)rows_idx[gc] : (int64_t)gc;
      p[j] = base + row * ld;
      ok[j] = in;
    }
  }
};

template <int ROWS, bool KC, typename T, int NT>
__device__ __forceinline__ void stage_load(Stage<ROWS, KC, T, NT>& s, const Rows<ROWS, KC, T, NT>& rw,
                                           const T* __restrict__ base, int64_t ld, int r0, int lim_row, int k0,
                                           int ke, const int32_t* rows_idx, int tid) {
#pragma unroll
  for (int j = 0; j < Stage<ROWS, KC, T, NT>::PER; ++j) {
    const int f = tid + NT * j;
    if (KC) {
      const int c = (f % (BK / 8)) * 8;
      s.u[j][0].load(rw.p[j], k0 + c, ke, rw.ok[j]);
    } else {
      const int kp = f / (ROWS / 8);       // k pair within the stage
      const int c = (f % (ROWS / 8)) * 8;  // 8 consecutive rows
      const int k = k0 + 2 * kp;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const bool ok = k + q < ke;
        const int kc = ok ? k + q : 0;
        const int64_t row = rows_idx ? (int64_t)rows_idx[kc] : (int64_t)kc;
        s.u[j][q].load(base + row * ld, r0 + c, lim_row, ok);
      }
    }
  }
}

template <int ROWS, bool KC, typename T, int NT>
__device__ __forceinline__ void stage_store(const Stage<ROWS, KC, T, NT>& s, uint16_t (*lds)[LDK], int tid) {
#pragma unroll
  for (int j = 0; j < Stage<ROWS, KC, T, NT>::PER; ++j) {
    const int f = tid + NT * j;
    if (KC) {
      const int rr = f / (BK / 8);
      const int c = (f % (BK / 8)) * 8;
      *reinterpret_cast<uint4*>(&lds[rr][c]) = s.u[j][0].packed();
    } else {
      const int kp = f / (ROWS / 8);
      const int c = (f % (ROWS / 8)) * 8;
      const uint4 lo4 = s.u[j][0].packed(), hi4 = s.u[j][1].packed();
      const uint32_t* lo = reinterpret_cast<const uint32_t*>(&lo4);
      const uint32_t* hi = reinterpret_cast<const uint32_t*>(&hi4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // elements 2e and 2e + 1 of the 8 rows, at k rows 2kp and 2kp + 1
        const uint32_t a = lo[e], b = hi[e];
        *reinterpret_cast<uint32_t*>(&lds[c + 2 * e][2 * kp]) = (a & 0xffffu) | (b << 16);
        *reinterpret_cast<uint32_t*>(&lds[c + 2 * e + 1][2 * kp]) = (a >> 16) | (b & 0xffff0000u);
      }
    }
  }
}

template <int BM, int BN, bool A_K, bool B_K, typename TA, typename TB>
__global__ void __launch_bounds__((BM / 64) * (BN / 64) * 64, 1) gemm_bf16s_kernel(Params p) {
  constexpr int WM = BM / 64, WN = BN / 64;
  constexpr int NT = WM * WN * 64;
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN][LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const ppo::TileCoord tc = ppo::xcd_tile();
  const int m0 = tc.m * BM;
  const int n0 = tc.n * BN;
  const int split = tc.z;
  const int kb = split * p.k_per_split;
  const int ke = min(p.K, kb + p.k_per_split);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float bsum[2] = {0.f, 0.f};
  const bool do_bsum = (p.bias_grad != nullptr) && (tc.m == 0) && (wm == 0);

  const TA* A = static_cast<const TA*>(p.A);
  const TB* B = static_cast<const TB*>(p.B);
  // two register sets, always addressed by compile-time index
  Stage<BM, A_K, TA, NT> sa0, sa1;
  Stage<BN, B_K, TB, NT> sb0, sb1;
  Rows<BM, A_K, TA, NT> ra;
  Rows<BN, B_K, TB, NT> rb;
  ra.init(A, p.lda, m0, p.M, p.rows, tid);
  rb.init(B, p.ldb, n0, p.N, nullptr, tid);
  auto load_a = [&](Stage<BM, A_K, TA, NT>& s, int k0) {
    stage_load(s, ra, A, p.lda, m0, p.M, k0, ke, p.rows, tid);
  };
  auto load_b = [&](Stage<BN, B_K, TB, NT>& s, int k0) {
    stage_load(s, rb, B, p.ldb, n0, p.N, k0, ke, nullptr, tid);
  };

  const int nk = (ke > kb) ? (ke - kb + BK - 1) / BK : 0;
  if (nk > 0) {
    load_a(sa0, kb);
    load_b(sb0, kb);
    if (nk > 1) {
      load_a(sa1, kb + BK);
      load_b(sb1, kb + BK);
    }
    stage_store(sa0, sA[0], tid);
    stage_store(sb0, sB[0], tid);
  }
  __syncthreads();

  auto mma_stage = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 a8[2], b8[2];
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
        a8[bi] = *reinterpret_cast<const bf16x8*>(&sA[buf][wm * 64 + bi * 32 + l32][kk + 8 * h]);
#pragma unroll
      for (int bj = 0; bj < 2; ++bj)
        b8[bj] = *reinterpret_cast<const bf16x8*>(&sB[buf][wn * 64 + bj * 32 + l32][kk + 8 * h]);
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
          acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8[bi], b8[bj], acc[bi][bj], 0, 0, 0);
      if (do_bsum) {
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
          float t = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) t += (float)b8[bj][e];
          bsum[bj] += t;
        }
      }
    }
  };

  // Stage kt is in LDS buffer kt & 1; stage kt + 1 in register set (kt + 1) & 1;
  // the loads of stage kt + 2 go to set kt & 1, free once stage kt was stored.
  for (int kt = 0; kt < nk; kt += 2) {
    if (kt + 2 < nk) {
      load_a(sa0, kb + (kt + 2) * BK);
      load_b(sb0, kb + (kt + 2) * BK);
    }
    mma_stage(0);
    if (kt + 1 < nk) {
      stage_store(sa1, sA[1], tid);
      stage_store(sb1, sB[1], tid);
    }
    __syncthreads();
    if (kt + 1 >= nk) break;
    if (kt + 3 < nk) {
      load_a(sa1, kb + (kt + 3) * BK);
      load_b(sb1, kb + (kt + 3) * BK);
    }
    mma_stage(1);
    if (kt + 2 < nk) {
      stage_store(sa0, sA[0], tid);
      stage_store(sb0, sB[0], tid);
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
  const bool rnd = p.round_out != 0;
  float* C = p.C + (int64_t)split * p.c_split_stride;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi) {
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
      const int gn = n0 + wn * 64 + bj * 32 + l32;
      const bool n_ok = gn < p.N;
      float bias = 0.f;
      if (p.epi == EPI_BIAS_ACT && p.bias && n_ok) bias = rnd ? bf16_round(p.bias[gn]) : p.bias[gn];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = m0 + wm * 64 + bi * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (!n_ok || gm >= p.M) continue;
        float v = acc[bi][bj][r];
        if (rnd) v = bf16_round(v);
        if (p.epi == EPI_BIAS_ACT) {
          if (p.bias) {
            v += bias;
            if (rnd) v = bf16_round(v);
          }
          if (p.act != ACT_NONE) {
            v = ppo::act_fwd(p.act, v);
            if (rnd) v = bf16_round(v);
          }
        } else if (p.epi == EPI_DACT) {
          v *= ppo::act_grad(p.act, p.aux[(int64_t)gm * p.ldaux + gn]);
          if (rnd) v = bf16_round(v);
        }
        C[(int64_t)gm * p.ldc + gn] = v;
      }
    }
  }
  if (do_bsum) {
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
      const float t = bsum[bj] + __shfl_xor(bsum[bj], 32, 64);
      const int gn = n0 + wn * 64 + bj * 32 + l32;
      if (h == 0 && gn < p.N) p.bias_grad[(int64_t)split * p.N + gn] = t;
    }
  }
}

template <int BM, int BN, bool A_K, bool B_K, typename TA, typename TB>
int launch(hipStream_t st, const Params& p, int splits) {
  dim3 grid(ppo::ceil_div(p.N, BN), ppo::ceil_div(p.M, BM), splits);
  hipLaunchKernelGGL((gemm_bf16s_kernel<BM, BN, A_K, B_K, TA, TB>), grid, dim3((BM / 64) * (BN / 64) * 64), 0, st,
                     p);
  return ppo::check_launch("ppo_gemm_bf16s");
}

template <bool A_K, bool B_K, typename TA, typename TB>
int launch_tile(hipStream_t st, const Params& p, int splits, int tile) {
  if (tile == 1) return launch<128, 128, A_K, B_K, TA, TB>(st, p, splits);
  return launch<256, 128, A_K, B_K, TA, TB>(st, p, splits);
}

template <bool A_K, bool B_K>
int launch_types(hipStream_t st, const Params& p, int splits, int tile, int a_bf16, int b_bf16) {
  if (a_bf16 && b_bf16) return launch_tile<A_K, B_K, uint16_t, uint16_t>(st, p, splits, tile);
  if (a_bf16) return launch_tile<A_K, B_K, uint16_t, float>(st, p, splits, tile);
  if (b_bf16) return launch_tile<A_K, B_K, float, uint16_t>(st, p, splits, tile);
  return launch_tile<A_K, B_K, float, float>(st, p, splits, tile);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

__global__ void cast_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
  const int64_t n8 = n / 8;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const floatx4 a = reinterpret_cast<const floatx4*>(x)[2 * i];
    const floatx4 b = reinterpret_cast<const floatx4*>(x)[2 * i + 1];
    uint4 v;
    v.x = pack2(a[0], a[1]);
    v.y = pack2(a[2], a[3]);
    v.z = pack2(b[0], b[1]);
    v.w = pack2(b[2], b[3]);
    reinterpret_cast<uint4*>(y)[i] = v;
  }
  for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = (uint16_t)bf16_bits(x[i]);
}

}  // namespace

// a_bf16 / b_bf16: the operand is stored as bf16 (uint16 bit patterns) rather
// than fp32.
// tile: -1 picks; 0: 256 x 128 (8 waves), 1: 128 x 128 (4 waves).
PPO_EXPORT int ppo_gemm_bf16s(void* stream, int a_layout, int b_layout, int a_bf16, int b_bf16, const void* A,
                              int64_t lda, const int32_t* rows, const void* B, int64_t ldb, float* C, int64_t ldc,
                              int M, int N, int K, int splits, int64_t c_split_stride, int epi, const float* bias,
                              int act, int round_out, const float* aux, int64_t ldaux, float* bias_grad, int tile) {
  if (M < 0 || N < 0 || K < 0 || splits < 1 || a_layout < 0 || a_layout > 1 || b_layout < 0 || b_layout > 1 ||
      epi < 0 || epi > 2 || act < 0 || act > 3 || tile > 1)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: bad argument (M=%d N=%d K=%d splits=%d)", M, N, K, splits);
  if (M == 0 || N == 0) return PPO_OK;
  if (!A || !B || !C) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: null operand");
  if (epi == EPI_DACT && !aux) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: EPI_DACT needs aux");
  if (bias_grad && !(a_layout == 1 && b_layout == 0))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: bias_grad needs a_layout=1, b_layout=0");
  if (splits > 1 && c_split_stride < (int64_t)M * ldc)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: split stride too small");
  // Every load is 16 bytes along the contiguous axis: rows must be 16-byte
  // aligned; an fp32 operand's contiguous extent a multiple of 4; a bf16
  // operand's row pitch at least its extent rounded up to 8 (the tail of a
  // row is read up to that pitch and masked).
  const int a_contig = a_layout == 0 ? K : M;
  const int b_contig = b_layout == 1 ? K : N;
  auto ok = [](const void* ptr, int64_t ld, int contig, int is_bf16) {
    if (!aligned16(ptr)) return false;
    if (is_bf16) return ld % 8 == 0 && ld >= (int64_t)((contig + 7) / 8 * 8);
    return ld % 4 == 0 && contig % 4 == 0;
  };
  if (!ok(A, lda, a_contig, a_bf16) || !ok(B, ldb, b_contig, b_bf16))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: operand rows must be 16-byte aligned with 16-byte vector "
                          "extents (lda=%lld ldb=%lld)", (long long)lda, (long long)ldb);
  Params p;
  p.A = A; p.lda = lda; p.rows = rows; p.B = B; p.ldb = ldb; p.C = C; p.ldc = ldc;
  p.c_split_stride = c_split_stride; p.M = M; p.N = N; p.K = K;
  p.k_per_split = ((ppo::ceil_div(K > 0 ? K : 1, splits) + BK - 1) / BK) * BK;
  p.epi = epi; p.bias = bias; p.act = act; p.round_out = round_out; p.aux = aux; p.ldaux = ldaux;
  p.bias_grad = bias_grad;
  if (tile < 0) tile = ((int64_t)ppo::ceil_div(M, 256) * ppo::ceil_div(N, 128) * splits >= 200) ? 0 : 1;
  hipStream_t st = ppo::as_stream(stream);
  if (a_layout == 0 && b_layout == 0) return launch_types<true, false>(st, p, splits, tile, a_bf16, b_bf16);
  if (a_layout == 0 && b_layout == 1) return launch_types<true, true>(st, p, splits, tile, a_bf16, b_bf16);
  if (a_layout == 1 && b_layout == 0) return launch_types<false, false>(st, p, splits, tile, a_bf16, b_bf16);
  return launch_types<false, true>(st, p, splits, tile, a_bf16, b_bf16);
}

// y[i] = bf16(x[i]) (round to nearest even), as 16-bit patterns; x, y 16-byte aligned.
PPO_EXPORT int ppo_cast_bf16(void* stream, const float* x, void* y, int64_t n) {
  if (n < 0 || (n > 0 && (!x || !y))) return ppo::set_error(PPO_ERR_ARG, "ppo_cast_bf16: bad argument");
  if (n == 0) return PPO_OK;
  if (!aligned16(x) || !aligned16(y)) return ppo::set_error(PPO_ERR_ARG, "ppo_cast_bf16: buffers must be 16-byte aligned");
  const int64_t blocks = std::min<int64_t>(ppo::ceil_div64(n / 8 + 1, 256), 8192);
  hipLaunchKernelGGL(cast_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, ppo::as_stream(stream), x,
                     static_cast<uint16_t*>(y), n);
  return ppo::check_launch("ppo_cast_bf16");
}
