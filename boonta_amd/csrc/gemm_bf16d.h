// The pipelined bf16 GEMM when both operands are stored as bf16 (the
// observation copy, the bf16 parameter image, bf16 cotangents): stages are
// copied from global memory straight into LDS by global_load_lds_dwordx4
// (each lane's 16 bytes land at the wave's LDS base + 16 * lane), so no
// registers hold staged data and no LDS store instructions run.  Contraction,
// layouts, row gather, split-K and epilogue are those of gemm_bf16s_kernel.
//
// LDS holds NBUF stages in a ring (3 for 256 x 128 tiles, 2 for 128 x 128,
// 2 for 256 x 256);
// stage kt + NBUF - 1 is issued right after the barrier that opens stage kt,
// so NBUF - 1 stages of loads are in flight behind the MFMAs.  Layouts (bf16, no padding, 16-byte chunks XOR-swizzled
// by the row so that transpose reads, 16-byte operand reads and the copies
// all spread over the LDS banks):
//   k-contiguous operand [ROWS][BK]: chunk c of row r at c ^ kc_swizzle(r);
//   k-outer operand [BK][ROWS]: chunk c of k row k at c ^ ko_swizzle(k).
// The swizzle is applied on the global side: lane l of a copy fetches the
// chunk whose swizzled position is its LDS slot.
//
// Ragged edges: rows beyond M / N are read from a clamped in-range row or
// column (finite data whose products only reach outputs that are not
// stored); a final stage cut short by K goes through registers with the
// elements past K zeroed.
#pragma once
#include "gemm_bf16s.h"

namespace ppo_bf16s {

constexpr int KIDX_MAX = 2048;  // reduction rows per split when the k-outer A operand is gathered
constexpr int KIDX_256 = 4096;  // the same for the 256 x 256 tile (its ring holds two stages)

using ppo::kc_swizzle;
__device__ __forceinline__ int ko_swizzle(int k) { return ((k & 1) ? 4 : 0) ^ ((k & 2) ? 10 : 0); }

__device__ __forceinline__ void copy16_to_lds(const uint16_t* src, uint16_t* lds_wave_base) {
  ppo::lds_copy16(src, lds_wave_base);
}
using ppo::stage_barrier;

// One operand's copies: ROWS x BK per stage in 1 KB copies (64 lanes x 16 B),
// PERW copies per wave.  For copy i of a wave, lane l fills LDS unit
// u = 64 (wave * PERW + i) + l.  KC: src is the (gathered) row, col the
// unit's k offset in the stage; k-outer: col is the unit's first element
// (clamped to the row's extent), rows come from the stage's k rows (through
// the block's LDS copy of the gather indices when the reduction is gathered).
template <int ROWS, bool KC, int NW, int SBK = BK>
struct DOperand {
  static_assert(SBK == BK || (!KC && (SBK == 32 || SBK == 16)),
                "a k-contiguous operand keeps 64-deep stages (its swizzle spans 8 chunks per row)");
  static constexpr int ELEMS = ROWS * SBK;
  static constexpr int COPIES = ELEMS / 512;
  static constexpr int PERW = COPIES / NW;
  static_assert(PERW >= 1 && COPIES % NW == 0, "tile too small for the wave count");
  static_assert(KC || ROWS >= 128, "k-outer swizzle needs 16 chunks per k row");
  const uint16_t* src[PERW];
  int krow[PERW];
  int col[PERW];
  bool ok[PERW];

  __device__ __forceinline__ void init(const uint16_t* base, int64_t ld, int r0, int lim, const int32_t* rows_idx,
                                       int wave, int lane) {
#pragma unroll
    for (int i = 0; i < PERW; ++i) {
      const int u = 64 * (wave * PERW + i) + lane;
      if (KC) {
        const int r = u / (SBK / 8);
        const int g = r0 + r;
        ok[i] = g < lim;
        const int gc = ok[i] ? g : 0;
        const int64_t row = rows_idx ? (int64_t)rows_idx[gc] : (int64_t)gc;
        src[i] = base + row * ld;
        col[i] = 8 * ((u % (SBK / 8)) ^ kc_swizzle(r));
        krow[i] = 0;
      } else {
        const int k = u / (ROWS / 8);
        const int c = (u % (ROWS / 8)) ^ ko_swizzle(k);
        const int last = ((lim - 1) / 8) * 8;  // the last 8-element unit holding valid elements
        src[i] = base;
        col[i] = min(r0 + 8 * c, last);
        krow[i] = k;
        ok[i] = true;
      }
    }
  }

  // k-outer row of reduction index k (kidx: the gather indices of the split
  // in LDS, from kb, or null)
  __device__ __forceinline__ int64_t krow_of(int k, int kb, const int32_t* kidx) const {
    return kidx ? (int64_t)kidx[k - kb] : (int64_t)k;
  }

  // Copies of the stage starting at k0 (entirely inside the split's range).
  __device__ __forceinline__ void copy(uint16_t* lds_stage, int64_t ld, int k0, int kb, const int32_t* kidx,
                                       int wave) const {
#pragma unroll
    for (int i = 0; i < PERW; ++i) {
      uint16_t* dst = lds_stage + 512 * (wave * PERW + i);
      if (KC) {
        copy16_to_lds(src[i] + k0 + col[i], dst);
      } else {
        copy16_to_lds(src[i] + krow_of(k0 + krow[i], kb, kidx) * ld + col[i], dst);
      }
    }
  }

  // The same units through registers, elements at k >= ke (and k-outer
  // columns >= lim) zeroed: a final stage cut short by K.
  __device__ __forceinline__ void copy_masked(uint16_t* lds_stage, int64_t ld, int k0, int ke, int lim, int kb,
                                              const int32_t* kidx, int wave, int lane) const {
    Unit<uint16_t> u[PERW];
#pragma unroll
    for (int i = 0; i < PERW; ++i) {
      if (KC) {
        u[i].load(src[i], k0 + col[i], ke, ok[i]);
      } else {
        const int k = k0 + krow[i];
        const bool in = k < ke;
        u[i].load(src[i] + krow_of(in ? k : k0, kb, kidx) * ld, col[i], lim, in);
      }
    }
#pragma unroll
    for (int i = 0; i < PERW; ++i)
      *reinterpret_cast<uint4*>(lds_stage + 512 * (wave * PERW + i) + 8 * lane) = u[i].packed();
  }
};

// MFMA operand (v_mfma_f32_32x32x16_bf16) for rows r0 .. r0 + 31, k kk .. kk + 15.
template <int ROWS, bool KC, int SBK = BK>
__device__ __forceinline__ bf16x8 doperand(const uint16_t* lds, int r0, int kk, int lane) {
  if (KC) {
    const int r = r0 + (lane & 31);
    const int c = (kk >> 3) + (lane >> 5);
    return *reinterpret_cast<const bf16x8*>(lds + r * SBK + ((c ^ kc_swizzle(r)) << 3));
  } else {
    const int g = lane >> 4, j = lane & 15;
    const int k = kk + 8 * (g >> 1) + (j >> 2);
    const int e = r0 + 16 * (g & 1) + 4 * (j & 3);
    const int off = k * ROWS + (((e >> 3) ^ ko_swizzle(k)) << 3) + (e & 4);  // k + 4 has the same swizzle
    typedef __attribute__((address_space(3))) uint16_t lds_u16;
    lds_u16* base = (lds_u16*)(lds);
    const shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(base + off));
    const shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(base + off + 4 * ROWS));
    const shortx8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, v);
  }
}

using ppo::ring_barrier;

// One workgroup's output tile tc of the GEMM p, SBK reduction elements per
// stage (64; 32 or 16 when both operands are k-outer, for a deeper ring in
// the same LDS).
template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, int NBUF, int KIDX, int SBK = BK>
__device__ __forceinline__ void gemm_bf16d_tile(const Params& p, const ppo::TileCoord tc) {
  constexpr int NW = WM * WN;
  constexpr int BI = BM / WM / 32, BJ = BN / WN / 32;
  static_assert(BI * WM * 32 == BM && BJ * WN * 32 == BN, "tile must split into 32 x 32 blocks");
  static_assert(BK % SBK == 0, "split boundaries (multiples of BK) must fall on stage boundaries");
  using OpA = DOperand<BM, A_K, NW, SBK>;
  using OpB = DOperand<BN, B_K, NW, SBK>;
  __shared__ __attribute__((aligned(1024))) uint16_t sA[NBUF][OpA::ELEMS];
  __shared__ __attribute__((aligned(1024))) uint16_t sB[NBUF][OpB::ELEMS];
  // gather indices of the split's reduction rows (A k-outer and gathered)
  __shared__ int32_t sIdx[A_K ? 1 : KIDX];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave % WM;
  const int wn = wave / WM;
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

  const uint16_t* A = static_cast<const uint16_t*>(p.A);
  const uint16_t* B = static_cast<const uint16_t*>(p.B);
  OpA oa;
  OpB ob;
  // A's gather applies to its rows (KC: m) or to the reduction rows (k-outer)
  oa.init(A, p.lda, m0, p.M, A_K ? p.rows : nullptr, wave, lane);
  ob.init(B, p.ldb, n0, p.N, nullptr, wave, lane);
  const int32_t* kidx = nullptr;
  if (!A_K && p.rows) {
    for (int i = threadIdx.x; i < ke - kb; i += NW * 64) sIdx[i] = p.rows[kb + i];
    kidx = sIdx;
    __syncthreads();
  }

  const int nk = (ke > kb) ? (ke - kb + SBK - 1) / SBK : 0;
  const int nfull = (ke - kb) / SBK;  // stages entirely inside [kb, ke)
  constexpr int PER_STAGE = OpA::PERW + OpB::PERW;  // copies a wave issues per stage

  auto issue = [&](int s) {  // stage s into ring slot s % NBUF
    uint16_t* la = sA[s % NBUF];
    uint16_t* lb = sB[s % NBUF];
    const int k0 = kb + s * SBK;
    if (s < nfull) {
      oa.copy(la, p.lda, k0, kb, kidx, wave);
      ob.copy(lb, p.ldb, k0, kb, nullptr, wave);
    } else {
      oa.copy_masked(la, p.lda, k0, ke, p.M, kb, kidx, wave, lane);
      ob.copy_masked(lb, p.ldb, k0, ke, p.N, kb, nullptr, wave, lane);
    }
  };

#pragma unroll
  for (int s = 0; s < NBUF - 1; ++s)
    if (s < nk) issue(s);

  auto mma_stage = [&](const uint16_t* la, const uint16_t* lb) {
    bf16x8 a8[2][BI], b8[2][BJ];
    auto read_ops = [&](int set, int kk) {
#pragma unroll
      for (int bi = 0; bi < BI; ++bi)
        a8[set][bi] = doperand<BM, A_K, SBK>(la, wm * (BI * 32) + bi * 32, kk, lane);
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj)
        b8[set][bj] = doperand<BN, B_K, SBK>(lb, wn * (BJ * 32) + bj * 32, kk, lane);
    };
    read_ops(0, 0);
#pragma unroll
    for (int ks = 0; ks < SBK / 16; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < SBK / 16) read_ops(cur ^ 1, (ks + 1) * 16);
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

  for (int kt = 0; kt < nk; ++kt) {
    // this wave's copies of stage kt are done once at most the younger
    // stages' copies are outstanding; the barrier then covers every wave's
    ring_barrier<PER_STAGE, NBUF - 2>(min(NBUF - 2, nk - 1 - kt));
    if (kt + NBUF - 1 < nk) issue(kt + NBUF - 1);  // the slot stage kt - 1 used
    mma_stage(sA[kt % NBUF], sB[kt % NBUF]);
  }

  epilogue<BI, BJ>(p, acc, bsum, do_bsum, m0 + wm * (BI * 32), n0 + wn * (BJ * 32), split, lane);
}

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, int NBUF, int KIDX = KIDX_MAX, int SBK = BK>
__global__ void __launch_bounds__(WM * WN * 64, 1) gemm_bf16d_kernel(Params p) {
  gemm_bf16d_tile<BM, BN, WM, WN, A_K, B_K, NBUF, KIDX, SBK>(p, ppo::xcd_tile());
}

// Several GEMMs of one tile shape in one launch: problem i owns the linear
// tiles [start[i], start[i + 1]), each problem's tiles ordered n fastest, then
// m, then split.  Linear tiles are dealt to the XCDs in contiguous ranges, as
// xcd_tile does for one GEMM.
constexpr int GROUP_MAX = 8;
struct GroupParams {
  Params p[GROUP_MAX];
  int start[GROUP_MAX + 1];
  int gx[GROUP_MAX], gy[GROUP_MAX];
  int count;
};

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, int NBUF, int KIDX, int SBK = BK>
__global__ void __launch_bounds__(WM * WN * 64, 1) gemm_bf16d_group_kernel(GroupParams g) {
  const int total = gridDim.x;
  const int w = blockIdx.x;
  const int x = w & 7, j = w >> 3;
  const int q = total >> 3, r = total & 7;
  const int t = x * q + (x < r ? x : r) + j;
  int i = 0;
  while (i + 1 < g.count && t >= g.start[i + 1]) ++i;
  const int local = t - g.start[i];
  ppo::TileCoord tc;
  tc.n = local % g.gx[i];
  tc.m = (local / g.gx[i]) % g.gy[i];
  tc.z = local / (g.gx[i] * g.gy[i]);
  gemm_bf16d_tile<BM, BN, WM, WN, A_K, B_K, NBUF, KIDX, SBK>(g.p[i], tc);
}

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, int NBUF, int KIDX = KIDX_MAX, int SBK = BK>
int launch_d(hipStream_t st, const Params& p, int splits) {
  dim3 grid(ppo::ceil_div(p.N, BN), ppo::ceil_div(p.M, BM), splits);
  hipLaunchKernelGGL((gemm_bf16d_kernel<BM, BN, WM, WN, A_K, B_K, NBUF, KIDX, SBK>), grid, dim3(WM * WN * 64), 0,
                     st, p);
  return ppo::check_launch("ppo_gemm_bf16s");
}

}  // namespace ppo_bf16s
