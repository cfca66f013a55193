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
//   - each operand keeps its memory orientation in LDS, so every global load
//     and every LDS store is 16 bytes along the contiguous axis.  A
//     k-contiguous operand ([row][k]) gives an MFMA operand (8 consecutive k
//     of one row) in one 16-byte LDS read; a k-outer operand ([k][row]) gives
//     it in two LDS transpose reads (ds_read_b64_tr_b16: within each group of
//     16 lanes, lane i receives element i % 4 of the 8-byte rows addressed by
//     lanes 4e + i / 4, e = 0..3).
#pragma once
#include <utility>
#include "common.h"

#include <algorithm>

// Kernel template of the pipelined bf16 GEMM; each operand storage pair
// (fp32 / bf16 for A and B) is instantiated in its own translation unit.
namespace ppo_bf16s {
constexpr int BK = 64;

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

// One operand's stage: ROWS (m or n) x BK, NT threads, as units of 8
// elements along the contiguous axis.  KC: memory is [row][k] (k
// contiguous); otherwise [k][row].
template <int ROWS, bool KC, typename T, int NT>
struct Stage {
  static constexpr int UNITS = ROWS * BK / 8;
  static constexpr int PER = UNITS / NT;
  static_assert(PER >= 1 && UNITS % NT == 0, "tile too small for the thread count");
  Unit<T> u[PER];
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
      s.u[j].load(rw.p[j], k0 + c, ke, rw.ok[j]);
    } else {
      const int k = k0 + f / (ROWS / 8);   // one k row
      const int c = (f % (ROWS / 8)) * 8;  // 8 consecutive rows of the operand
      const bool ok = k < ke;
      const int kc = ok ? k : 0;
      const int64_t row = rows_idx ? (int64_t)rows_idx[kc] : (int64_t)kc;
      s.u[j].load(base + row * ld, r0 + c, lim_row, ok);
    }
  }
}

// LDS layouts (bf16 elements).  KC: [ROWS][BK], the 16-byte k group kg of
// row r stored at group kg ^ sw(r), sw a linear (XOR) map of the row's low
// five bits chosen so that neither the 16-byte stores (8 lanes per row) nor
// the MFMA operand reads (32 consecutive rows, two groups) put two lanes of a
// bank phase on one bank.  k-outer: [BK][ROWS + TPAD]; the pad spreads the
// 4 consecutive k rows one transpose read touches over the banks.
#ifndef PPO_BF16S_NSET
#define PPO_BF16S_NSET 2  // register stage sets when both operands are stored as bf16
#endif
#ifndef PPO_BF16S_TPAD
#define PPO_BF16S_TPAD 16
#endif
constexpr int TPAD = PPO_BF16S_TPAD;

template <int ROWS, bool KC>
struct Lds {
  static constexpr int PITCH = KC ? BK : ROWS + TPAD;
  static constexpr int ELEMS = KC ? ROWS * BK : BK * (ROWS + TPAD);
};

__device__ __forceinline__ int swz(int row, int kg) {
  const int sw = (row & 3) ^ ((row & 4) ? 5 : 0) ^ ((row & 8) ? 3 : 0) ^ ((row & 16) ? 4 : 0);
  return (kg ^ sw) << 3;
}

template <int ROWS, bool KC, typename T, int NT>
__device__ __forceinline__ void stage_store(const Stage<ROWS, KC, T, NT>& s, uint16_t* lds, int tid) {
#pragma unroll
  for (int j = 0; j < Stage<ROWS, KC, T, NT>::PER; ++j) {
    const int f = tid + NT * j;
    int off;
    if (KC) {
      const int rr = f / (BK / 8);
      off = rr * BK + swz(rr, f % (BK / 8));
    } else {
      off = (f / (ROWS / 8)) * Lds<ROWS, false>::PITCH + (f % (ROWS / 8)) * 8;
    }
    *reinterpret_cast<uint4*>(lds + off) = s.u[j].packed();
  }
}

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

// MFMA operand of v_mfma_f32_32x32x16_bf16 for rows r0 .. r0 + 31 and k
// kk .. kk + 15 (lane l: row r0 + l % 32, k kk + 8 (l / 32) .. + 7).
template <int ROWS, bool KC>
__device__ __forceinline__ bf16x8 operand(const uint16_t* lds, int r0, int kk, int lane) {
  if (KC) {
    const int r = r0 + (lane & 31);
    return *reinterpret_cast<const bf16x8*>(lds + r * BK + swz(r, (kk >> 3) + (lane >> 5)));
  } else {
    // lane j of 16-lane group g points at k row kk + 8 (g / 2) + j / 4 (+ 4),
    // rows r0 + 16 (g % 2) + 4 (j % 4) .. + 3; it receives its own row's 4 k
    constexpr int P = Lds<ROWS, false>::PITCH;
    const int g = lane >> 4, j = lane & 15;
    const int off = (kk + 8 * (g >> 1) + (j >> 2)) * P + r0 + 16 * (g & 1) + 4 * (j & 3);
    typedef __attribute__((address_space(3))) uint16_t lds_u16;
    lds_u16* base = (lds_u16*)(lds);
    const shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(base + off));
    const shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(base + off + 4 * P));
    const shortx8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, v);
  }
}

// One 32 x 32 block (rows wm0b.., columns wn0b..) of the epilogue.  EPI_ /
// ACT_: the epilogue kind and activation when the launch fixes them at
// compile time (the unrolled element loop then holds only their code), -1
// for the run-time values.
template <int EPI_, int ACT_>
__device__ __forceinline__ void epilogue_block(const Params& p, float* C, const floatx16& a, int wm0b, int wn0b,
                                               int h, int l32) {
  const int epi = EPI_ >= 0 ? EPI_ : p.epi;
  const int act = ACT_ >= 0 ? ACT_ : p.act;
  const bool rnd = p.round_out != 0;
  const int gn = wn0b + l32;
  const bool n_ok = gn < p.N;
  float bias = 0.f;
  if (epi == EPI_BIAS_ACT && p.bias && n_ok) bias = rnd ? bf16_round(p.bias[gn]) : p.bias[gn];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int gm = wm0b + 8 * (r >> 2) + 4 * h + (r & 3);
    if (!n_ok || gm >= p.M) continue;
    float v = a[r];
    if (rnd) v = bf16_round(v);
    if (epi == EPI_BIAS_ACT) {
      if (p.bias) {
        v += bias;
        if (rnd) v = bf16_round(v);
      }
      if (act != ACT_NONE) {
        v = ppo::act_fwd(act, v);
        if (rnd) v = bf16_round(v);
      }
    } else if (epi == EPI_DACT) {
      v *= ppo::act_grad(act, p.aux[(int64_t)gm * p.ldaux + gn]);
      if (rnd) v = bf16_round(v);
    }
    C[(int64_t)gm * p.ldc + gn] = v;
  }
}

template <int EPI_, int ACT_, int BI, int BJ, int... I>
__device__ __forceinline__ void epilogue_blocks(const Params& p, float* C, floatx16 (&acc)[BI][BJ], int wm0, int wn0,
                                                int h, int l32, std::integer_sequence<int, I...>) {
  // compile-time block indices: the accumulators stay in registers
  (epilogue_block<EPI_, ACT_>(p, C, acc[I / BJ][I % BJ], wm0 + (I / BJ) * 32, wn0 + (I % BJ) * 32, h, l32), ...);
}

// The wave's BI x BJ accumulator blocks (rows from wm0, columns from wn0)
// with the epilogue, and the bias-gradient column sums of B.
template <int BI, int BJ>
__device__ __forceinline__ void epilogue(const Params& p, floatx16 (&acc)[BI][BJ], const float (&bsum)[BJ],
                                         bool do_bsum, int wm0, int wn0, int split, int lane) {
  const int h = lane >> 5;
  const int l32 = lane & 31;
  float* C = p.C + (int64_t)split * p.c_split_stride;
  // the workloads' epilogues as compile-time constants; others at run time
  const auto seq = std::make_integer_sequence<int, BI * BJ>{};
  if (p.epi == EPI_STORE)
    epilogue_blocks<EPI_STORE, ACT_NONE, BI, BJ>(p, C, acc, wm0, wn0, h, l32, seq);
  else if (p.epi == EPI_BIAS_ACT && p.act == ACT_RELU)
    epilogue_blocks<EPI_BIAS_ACT, ACT_RELU, BI, BJ>(p, C, acc, wm0, wn0, h, l32, seq);
  else if (p.epi == EPI_DACT && p.act == ACT_RELU)
    epilogue_blocks<EPI_DACT, ACT_RELU, BI, BJ>(p, C, acc, wm0, wn0, h, l32, seq);
  else
    epilogue_blocks<-1, -1, BI, BJ>(p, C, acc, wm0, wn0, h, l32, seq);
  if (do_bsum) {
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj) {
      const float t = ppo::add_xor32(bsum[bj]);
      const int gn = wn0 + bj * 32 + l32;
      if (h == 0 && gn < p.N) p.bias_grad[(int64_t)split * p.N + gn] = t;
    }
  }
}

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, typename TA, typename TB>
__global__ void __launch_bounds__(WM * WN * 64, 1) gemm_bf16s_kernel(Params p) {
  constexpr int NT = WM * WN * 64;
  constexpr int BI = BM / WM / 32, BJ = BN / WN / 32;  // 32 x 32 blocks per wave
  static_assert(BI * WM * 32 == BM && BJ * WN * 32 == BN, "tile must split into 32 x 32 blocks");
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][Lds<BM, A_K>::ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][Lds<BN, B_K>::ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  const ppo::TileCoord tc = ppo::xcd_tile();
  const int m0 = tc.m * BM;
  const int n0 = tc.n * BN;
  const int split = tc.z;
  const int kb = split * p.k_per_split;
  const int ke = min(p.K, kb + p.k_per_split);

  floatx16 acc[BI][BJ];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int j = 0; j < BJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float bsum[BJ];
#pragma unroll
  for (int j = 0; j < BJ; ++j) bsum[j] = 0.f;
  const bool do_bsum = (p.bias_grad != nullptr) && (tc.m == 0) && (wm == 0);

  const TA* A = static_cast<const TA*>(p.A);
  const TB* B = static_cast<const TB*>(p.B);
  // NSET register sets of staged loads, always addressed by compile-time
  // index: the loads of stage k + 1 are issued NSET stages before their LDS
  // store (NSET even, so LDS buffer k & 1 follows the set index's parity)
  constexpr int NSET = (sizeof(TA) == 2 && sizeof(TB) == 2) ? PPO_BF16S_NSET : 2;
  static_assert(NSET % 2 == 0, "NSET must be even");
  Stage<BM, A_K, TA, NT> sa[NSET];
  Stage<BN, B_K, TB, NT> sb[NSET];
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
#pragma unroll
  for (int s = 0; s < NSET; ++s) {
    if (s < nk) {
      load_a(sa[s], kb + s * BK);
      load_b(sb[s], kb + s * BK);
    }
  }
  if (nk > 0) {
    stage_store(sa[0], sA[0], tid);
    stage_store(sb[0], sB[0], tid);
  }
  if (NSET < nk) {  // set 0 is free again: stage NSET
    load_a(sa[0], kb + NSET * BK);
    load_b(sb[0], kb + NSET * BK);
  }
  __syncthreads();

  // The operands of k step kk + 16 are read from LDS while the MFMAs of step
  // kk run (two operand register sets), so LDS latency hides behind them.
  auto mma_stage = [&](int buf) {
    bf16x8 a8[2][BI], b8[2][BJ];
    auto read_ops = [&](int set, int kk) {
#pragma unroll
      for (int bi = 0; bi < BI; ++bi)
        a8[set][bi] = operand<BM, A_K>(sA[buf], wm * (BI * 32) + bi * 32, kk, lane);
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
        b8[set][bj] = operand<BN, B_K>(sB[buf], wn * (BJ * 32) + bj * 32, kk, lane);
    };
    read_ops(0, 0);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < BK / 16) read_ops(cur ^ 1, (ks + 1) * 16);
#pragma unroll
      for (int bi = 0; bi < BI; ++bi)
#pragma unroll
        for (int bj = 0; bj < BJ; ++bj)
          acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8[cur][bi], b8[cur][bj], acc[bi][bj], 0, 0, 0);
      if (do_bsum) {
#pragma unroll
        for (int bj = 0; bj < BJ; ++bj) {
          float t = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) t += (float)b8[cur][bj][e];
          bsum[bj] += t;
        }
      }
    }
  };

  // Stage kt sits in LDS buffer kt & 1 and was staged in set kt % NSET.
  // After its MFMAs, stage kt + 1 goes from its set to the other buffer and
  // the set is refilled with stage kt + 1 + NSET.
  for (int kt0 = 0; kt0 < nk; kt0 += NSET) {
#pragma unroll
    for (int s = 0; s < NSET; ++s) {
      const int kt = kt0 + s;
      if (kt < nk) {
        mma_stage(s & 1);
        const int nx = (s + 1) % NSET;
        if (kt + 1 < nk) {
          stage_store(sa[nx], sA[(s + 1) & 1], tid);
          stage_store(sb[nx], sB[(s + 1) & 1], tid);
        }
        if (kt + 1 + NSET < nk) {
          load_a(sa[nx], kb + (kt + 1 + NSET) * BK);
          load_b(sb[nx], kb + (kt + 1 + NSET) * BK);
        }
        __syncthreads();
      }
    }
  }

  epilogue<BI, BJ>(p, acc, bsum, do_bsum, m0 + wm * (BI * 32), n0 + wn * (BJ * 32), split, lane);
}

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, typename TA, typename TB>
int launch(hipStream_t st, const Params& p, int splits) {
  dim3 grid(ppo::ceil_div(p.N, BN), ppo::ceil_div(p.M, BM), splits);
  hipLaunchKernelGGL((gemm_bf16s_kernel<BM, BN, WM, WN, A_K, B_K, TA, TB>), grid, dim3(WM * WN * 64), 0, st, p);
  return ppo::check_launch("ppo_gemm_bf16s");
}

template <bool A_K, bool B_K, typename TA, typename TB>
int launch_tile(hipStream_t st, const Params& p, int splits, int tile) {
  // Wave tiles of 64 x 64: larger ones (128 x 64 and up) spill the two
  // staged register sets to scratch.
  if (tile == 1) return launch<128, 128, 2, 2, A_K, B_K, TA, TB>(st, p, splits);
  return launch<256, 128, 4, 2, A_K, B_K, TA, TB>(st, p, splits);
}

// Every layout of one operand storage pair (defined in gemm_bf16s_<ta><tb>.hip).
template <typename TA, typename TB>
int launch_layouts(hipStream_t st, const Params& p, int splits, int tile, int a_layout, int b_layout);
template <>
int launch_layouts<float, float>(hipStream_t, const Params&, int, int, int, int);
template <>
int launch_layouts<float, uint16_t>(hipStream_t, const Params&, int, int, int, int);
template <>
int launch_layouts<uint16_t, float>(hipStream_t, const Params&, int, int, int, int);
template <>
int launch_layouts<uint16_t, uint16_t>(hipStream_t, const Params&, int, int, int, int);

template <typename TA, typename TB>
int launch_layouts_impl(hipStream_t st, const Params& p, int splits, int tile, int a_layout, int b_layout) {
  if (a_layout == 0 && b_layout == 0) return launch_tile<true, false, TA, TB>(st, p, splits, tile);
  if (a_layout == 0 && b_layout == 1) return launch_tile<true, true, TA, TB>(st, p, splits, tile);
  if (a_layout == 1 && b_layout == 0) return launch_tile<false, false, TA, TB>(st, p, splits, tile);
  return launch_tile<false, true, TA, TB>(st, p, splits, tile);
}

}  // namespace ppo_bf16s
