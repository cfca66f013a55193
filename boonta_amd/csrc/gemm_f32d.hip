// fp32 GEMM fed by direct global -> LDS copies (global_load_lds_dwordx4: each
// lane's 16 bytes land at the wave's LDS base + 16 * lane), for operands with
// 16-byte rows along their contiguous axis.  Same contraction, layouts, row
// gather, split-K and epilogues as the register-staged kernel in gemm.hip;
// no registers hold staged data and no LDS store instructions run.  The
// 4-wave tiles keep a ring of two stages (the copies of the next stage in
// flight behind the MFMAs of this one): the smaller LDS footprint keeps more
// workgroups resident per CU, which hides the L2 latency better than a third
// stage does (LDS allows five 64 x 64 workgroups per CU instead of three, two
// 128 x 128 instead of one).  The 8-wave tiles keep three.
//
// Tiles: 4 wave64s in 2 x 2 (64 / 128 x 64 / 128 tiles) or 8 in 2 x 4 / 4 x 2
// (128 x 256, 256 x 128), each wave (BM/WM) x (BN/WN) of 32 x 32 blocks of
// v_mfma_f32_32x32x2_f32; 32 reduction elements per stage.  The 8-wave tiles
// read 2-4x fewer operand bytes per FLOP from L2 (a 64 x 64 tile at full fp32
// MFMA rate needs more L2 bandwidth than the chip has).  Inside each group of
// 8 reduction elements, lane half h consumes k = 8g + 4h + s at MFMA step s
// (both operands use the same order, so the sum is unchanged).
// LDS layouts (fp32, 16-byte chunks XOR-swizzled on the copy side):
//   k-contiguous [ROWS][32]: chunk c of row r at c ^ kc_swizzle(r); an operand
//     read (4 consecutive k of one row) is one 16-byte read;
//   k-outer [32][ROWS]: chunk c of k row k at c ^ (8 * bit 2 of k), so the two
//     lane halves (k and k + 4) read different bank halves.
// Ragged edges: rows beyond M / N are read from a clamped in-range row or
// column (only outputs that are not stored see them); a final stage cut short
// by K goes through registers with the elements past K zeroed.
#include "gemm_f32.h"
#include "grad_reduce.h"

namespace ppo_f32 {
namespace {

constexpr int BK = F32D_BK;

__device__ __forceinline__ int ko_swizzle32(int k) { return ((k >> 2) & 1) << 3; }

// One operand's copies: ROWS x BK fp32 per stage in 1 KB copies (64 lanes x
// 16 B), PERW per wave (NW waves); copy i of a wave fills LDS units
// 64 (wave PERW + i) + l.
template <int ROWS, bool KC, int NW>
struct Operand {
  static constexpr int ELEMS = ROWS * BK;
  static constexpr int COPIES = ELEMS / 256;
  static constexpr int PERW = COPIES / NW;
  static_assert(PERW >= 1 && COPIES % NW == 0, "tile too small for the wave count");
  static_assert(KC || ROWS >= 64, "k-outer swizzle needs 16 chunks per k row");
  const float* src[PERW];  // KC: the (gathered) row; k-outer: the operand base
  int col[PERW];           // KC: the unit's k offset in the stage; k-outer: its first element (clamped)
  int krow[PERW];          // k-outer: the unit's k row in the stage
  bool ok[PERW];           // KC: row in range

  __device__ __forceinline__ void init(const float* base, int64_t ld, int r0, int lim, const int32_t* rows_idx,
                                       int wave, int lane) {
#pragma unroll
    for (int i = 0; i < PERW; ++i) {
      const int u = 64 * (wave * PERW + i) + lane;
      if (KC) {
        const int r = u / (BK / 4);
        const int g = r0 + r;
        ok[i] = g < lim;
        const int gc = ok[i] ? g : 0;
        const int64_t row = rows_idx ? (int64_t)rows_idx[gc] : (int64_t)gc;
        src[i] = base + row * ld;
        col[i] = 4 * ((u % (BK / 4)) ^ ppo::kc_swizzle(r));
        krow[i] = 0;
      } else {
        const int k = u / (ROWS / 4);
        const int c = (u % (ROWS / 4)) ^ ko_swizzle32(k);
        const int last = ((lim - 1) / 4) * 4;
        src[i] = base;
        col[i] = min(r0 + 4 * c, last);
        krow[i] = k;
        ok[i] = true;
      }
    }
  }

  __device__ __forceinline__ int64_t row_of(int k, int kb, const int32_t* kidx) const {
    return kidx ? (int64_t)kidx[k - kb] : (int64_t)k;
  }

  __device__ __forceinline__ void copy(float* lds_stage, int64_t ld, int k0, int kb, const int32_t* kidx,
                                       int wave) const {
#pragma unroll
    for (int i = 0; i < PERW; ++i) {
      float* dst = lds_stage + 256 * (wave * PERW + i);
      if (KC)
        ppo::lds_copy16(src[i] + k0 + col[i], dst);
      else
        ppo::lds_copy16(src[i] + row_of(k0 + krow[i], kb, kidx) * ld + col[i], dst);
    }
  }

  // Registers, elements at k >= ke (k-outer: also columns >= lim) zeroed.
  __device__ __forceinline__ void copy_masked(float* lds_stage, int64_t ld, int k0, int ke, int lim, int kb,
                                              const int32_t* kidx, int wave, int lane) const {
    floatx4 v[PERW];
#pragma unroll
    for (int i = 0; i < PERW; ++i) {
      if (KC) {
        const int k = k0 + col[i];
        const bool in = ok[i] && k < ke;
        v[i] = *reinterpret_cast<const floatx4*>(src[i] + (in ? k : 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][e] = (in && k + e < ke) ? v[i][e] : 0.f;
      } else {
        const int k = k0 + krow[i];
        const bool in = k < ke;
        v[i] = *reinterpret_cast<const floatx4*>(src[i] + row_of(in ? k : k0, kb, kidx) * ld + col[i]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][e] = (in && col[i] + e < lim) ? v[i][e] : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < PERW; ++i)
      *reinterpret_cast<floatx4*>(lds_stage + 256 * (wave * PERW + i) + 4 * lane) = v[i];
  }
};

// Operand values of 32 rows from rbase for reduction group g: element s is
// the value at k = 8g + 4h + s of row rbase + l32.
template <int ROWS, bool KC>
__device__ __forceinline__ floatx4 operand(const float* lds, int rbase, int g, int lane) {
  const int h = lane >> 5;
  const int r = rbase + (lane & 31);
  if (KC) {
    const int c = 2 * g + h;
    return *reinterpret_cast<const floatx4*>(lds + r * BK + ((c ^ ppo::kc_swizzle(r)) << 2));
  } else {
    floatx4 v;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = 8 * g + 4 * h + s;
      v[s] = lds[k * ROWS + ((((r >> 2) ^ ko_swizzle32(k))) << 2) + (r & 3)];
    }
    return v;
  }
}

// One BM x BN output tile (tile row tm, column tn) of split `split` of the
// GEMM p.
// KIDX: the LDS capacity for a gathered k-outer A's split indices.
// WT: a weight-gradient store whose partials another workgroup of the launch
// sums (EPI_STORE only; device-coherent stores).
template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, int NBUF, int KIDX = F32D_KIDX_MAX, bool WT = false>
__device__ __forceinline__ void gemm_f32d_tile(const GemmParams& p, int tm, int tn, int split) {
  constexpr int NW = WM * WN;
  constexpr int MB = BM / WM / 32, NB = BN / WN / 32;  // 32 x 32 blocks per wave
  static_assert(MB * WM * 32 == BM && NB * WN * 32 == BN, "tile must split into 32 x 32 blocks");
  using OpA = Operand<BM, A_K, NW>;
  using OpB = Operand<BN, B_K, NW>;
  __shared__ __attribute__((aligned(1024))) float sA[NBUF][OpA::ELEMS];
  __shared__ __attribute__((aligned(1024))) float sB[NBUF][OpB::ELEMS];
  __shared__ int32_t sIdx[A_K ? 1 : KIDX];  // gather indices of the split (k-outer A)

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave % WM;
  const int wn = wave / WM;
  const int m0 = tm * BM;
  const int n0 = tn * BN;
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
  const bool do_bsum = (p.bias_grad != nullptr) && (tm == 0) && (wm == 0);

  // The epilogue's inputs are loaded before the main loop (clamped rows /
  // columns read in-range data for outputs that are not stored), so the
  // epilogue does not wait on them.  Only in the layouts of the
  // input-cotangent GEMM (A k-contiguous, B = W read as [N][K]; one 32 x 32
  // block per wave: EPI_DACT's 16 aux values per lane) and of the forward
  // (A k-contiguous, B k-outer: EPI_BIAS_ACT's bias of each block column; the
  // 64 x 64 and 8-wave tiles), so no other instance holds registers for them.
  constexpr bool PRE_DACT = MB * NB == 1 && A_K && B_K;
  constexpr bool PRE_BIAS = A_K && !B_K && (MB * NB == 1 || NW == 8);  // the others would lose occupancy
  float auxv[MB * NB * 16];
  bool pre_aux = false;
  const int gn_pre = min(n0 + wn * (BN / WN) + (lane & 31), p.N - 1);
  if constexpr (PRE_DACT) {
    pre_aux = p.epi == EPI_DACT && p.aux != nullptr;
    if (pre_aux) {
      const int h = lane >> 5;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = min(m0 + wm * (BM / WM) + 8 * (r >> 2) + 4 * h + (r & 3), p.M - 1);
        auxv[r] = p.aux[(int64_t)gm * p.ldaux + gn_pre];
      }
    }
  }
  if constexpr (PRE_BIAS) {
    pre_aux = p.epi == EPI_BIAS_ACT && p.bias != nullptr;
    if (pre_aux) {
#pragma unroll
      for (int bj = 0; bj < NB; ++bj) auxv[bj] = p.bias[min(n0 + wn * (BN / WN) + bj * 32 + (lane & 31), p.N - 1)];
    }
  }

  OpA oa;
  OpB ob;
  oa.init(p.A, p.lda, m0, p.M, A_K ? p.rows : nullptr, wave, lane);
  ob.init(p.B, p.ldb, n0, p.N, nullptr, wave, lane);
  const int32_t* kidx = nullptr;
  if (!A_K && p.rows) {
    for (int i = threadIdx.x; i < ke - kb; i += NW * 64) sIdx[i] = p.rows[kb + i];
    kidx = sIdx;
    __syncthreads();
  }

  const int nk = (ke > kb) ? (ke - kb + BK - 1) / BK : 0;
  const int nfull = (ke - kb) / BK;
  constexpr int PER_STAGE = OpA::PERW + OpB::PERW;

  auto issue = [&](int s) {
    float* la = sA[s % NBUF];
    float* lb = sB[s % NBUF];
    const int k0 = kb + s * BK;
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

  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk)
      ppo::stage_barrier<PER_STAGE * (NBUF - 2)>();
    else
      ppo::stage_barrier<0>();
    if (kt + NBUF - 1 < nk) issue(kt + NBUF - 1);
    const float* la = sA[kt % NBUF];
    const float* lb = sB[kt % NBUF];
    floatx4 a4[2][MB], b4[2][NB];
    auto read_ops = [&](int set, int g) {
#pragma unroll
      for (int bi = 0; bi < MB; ++bi) a4[set][bi] = operand<BM, A_K>(la, wm * (BM / WM) + bi * 32, g, lane);
#pragma unroll
      for (int bj = 0; bj < NB; ++bj) b4[set][bj] = operand<BN, B_K>(lb, wn * (BN / WN) + bj * 32, g, lane);
    };
    read_ops(0, 0);
#pragma unroll
    for (int g = 0; g < BK / 8; ++g) {
      const int cur = g & 1;
      if (g + 1 < BK / 8) read_ops(cur ^ 1, g + 1);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int bi = 0; bi < MB; ++bi)
#pragma unroll
          for (int bj = 0; bj < NB; ++bj)
            acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[cur][bi][s], b4[cur][bj][s], acc[bi][bj], 0, 0, 0);
      if (do_bsum) {
#pragma unroll
        for (int bj = 0; bj < NB; ++bj)
          bsum[bj] += (b4[cur][bj][0] + b4[cur][bj][1]) + (b4[cur][bj][2] + b4[cur][bj][3]);
      }
    }
  }

  if constexpr (WT)
    epilogue_f32_t<MB, NB, EPI_STORE, ACT_NONE, false, true>(p, acc, bsum, do_bsum, m0 + wm * (BM / WM),
                                                             n0 + wn * (BN / WN), split, lane, auxv);
  else if (pre_aux)
    epilogue_f32<MB, NB, true>(p, acc, bsum, do_bsum, m0 + wm * (BM / WM), n0 + wn * (BN / WN), split, lane, auxv);
  else
    epilogue_f32<MB, NB>(p, acc, bsum, do_bsum, m0 + wm * (BM / WM), n0 + wn * (BN / WN), split, lane, auxv);
}

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, int NBUF>
__global__ void __launch_bounds__(WM * WN * 64) gemm_f32d_kernel(GemmParams p0) {
  const ppo::TileCoord tc = ppo::xcd_tile();
  const int tower = tc.z / p0.splits;
  const int split = tc.z - tower * p0.splits;
  gemm_f32d_tile<BM, BN, WM, WN, A_K, B_K, NBUF>(tower_params(p0, tower), tc.m, tc.n, split);
}

// Several GEMMs of one tile shape in one launch: problem i owns the linear
// tiles [start[i], start[i + 1]), ordered n fastest, then m, then split;
// linear tiles are dealt to the XCDs in contiguous ranges, as xcd_tile does
// for one GEMM.
template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, int NBUF>
__global__ void __launch_bounds__(WM * WN * 64) gemm_f32d_group_kernel(F32Group g) {
  const int total = gridDim.x;
  const int w = blockIdx.x;
  const int x = w & 7, j = w >> 3;
  const int q = total >> 3, r = total & 7;
  const int t = x * q + (x < r ? x : r) + j;
  int i = 0;
  while (i + 1 < g.count && t >= g.start[i + 1]) ++i;
  const int local = t - g.start[i];
  gemm_f32d_tile<BM, BN, WM, WN, A_K, B_K, NBUF>(g.p[i], (local / g.gx[i]) % g.gy[i], local % g.gx[i],
                                                 local / (g.gx[i] * g.gy[i]));
}

// The split-K counts the finishing sum is compiled for.
#define PPO_F32_FINAL_PARTS(X) X(1) X(2) X(3) X(4) X(6) X(8) X(12) X(16)

template <int BM, int BN, int WM, int WN, int NBUF, int KIDX>
__global__ void __launch_bounds__(WM * WN * 64) gemm_f32d_group_final_kernel(F32Group g, ppo_gr::DwFinal f) {
  static_assert(BM == 64 && BN == 64 && WM * WN == 4, "the finishing sum assumes 64 x 64 tiles of 4 waves");
  __shared__ floatx4 s_part[4][64];
  __shared__ double s_w[4];
  __shared__ int s_last;
  // the tiles first, then the workgroups of the other segments (whose
  // partials are complete before this launch): dispatched behind the tiles,
  // they do not hold back the tiles' start
  const int total = gridDim.x - f.rpad;
  if ((int)blockIdx.x >= total) {
    const int b = (int)blockIdx.x - total;
    if (b < f.rblocks)
      ppo_gr::reduce_block(b, static_cast<const ppo_gr::Segment*>(f.segs),
                           static_cast<const ppo_gr::Chunk*>(f.chunks), f.nchunks, f.nfew, f.nwide, f.sumsq, s_part);
    return;
  }
  // tiles as in gemm_f32d_group_kernel
  const int w = blockIdx.x;
  const int x = w & 7, j = w >> 3;
  const int q = total >> 3, r = total & 7;
  const int t = x * q + (x < r ? x : r) + j;
  int i = 0;
  while (i + 1 < g.count && t >= g.start[i + 1]) ++i;
  const GemmParams& p = g.p[i];
  const int local = t - g.start[i];
  const int tm = (local / g.gx[i]) % g.gy[i], tn = local % g.gx[i];
  gemm_f32d_tile<BM, BN, WM, WN, false, false, NBUF, KIDX, true>(p, tm, tn, local / (g.gx[i] * g.gy[i]));
  // every wave's partial stores complete, then one arrival for the tile
  const int slot = f.slot0[i] + tm * g.gx[i] + tn;
  double sq = 0.0;
  if (p.splits == 32 || p.splits == 64) {
    // two levels: the last of each group of eight splits sums the group,
    // the last group the group sums
    const int grp = (local / (g.gx[i] * g.gy[i])) >> 3;
    if (!ppo_gr::arrive_last(f.counters + f.ntiles + 8 * slot + grp, 8, &s_last)) return;
    ppo_gr::finish_group8<BM, BN, WM * WN * 64>(p.C, p.ldc, p.c_split_stride, f.g_rows[i], p.N, tm, tn, grp,
                                                p.bias_grad);
    if (!ppo_gr::arrive_last(f.counters + slot, p.splits / 8, &s_last)) return;
    if (p.splits == 32)
      sq = ppo_gr::finish_level2<BM, BN, WM * WN * 64, 4>(p.C, p.ldc, p.c_split_stride, f.g_rows[i], p.N, tm, tn,
                                                          f.G[i], f.ldg[i], p.bias_grad, f.Gb[i]);
    else
      sq = ppo_gr::finish_level2<BM, BN, WM * WN * 64, 8>(p.C, p.ldc, p.c_split_stride, f.g_rows[i], p.N, tm, tn,
                                                          f.G[i], f.ldg[i], p.bias_grad, f.Gb[i]);
    ppo_gr::block_sumsq<WM * WN * 64>(sq, s_w, f.sumsq + slot);
    return;
  }
  if (!ppo_gr::arrive_last(f.counters + slot, p.splits, &s_last)) return;
  switch (p.splits) {
#define PPO_F32_FINAL_CASE(S)                                                                                     \
  case S:                                                                                                         \
    sq = ppo_gr::finish_tile_sum<BM, BN, WM * WN * 64, S, 16>(p.C, p.ldc, p.c_split_stride, f.g_rows[i], p.N, tm, \
                                                              tn, f.G[i] + 0, f.ldg[i], false, p.bias_grad,      \
                                                              f.Gb[i]);                                           \
    break;
    PPO_F32_FINAL_PARTS(PPO_F32_FINAL_CASE)
#undef PPO_F32_FINAL_CASE
    default: break;  // rejected by the host
  }
  ppo_gr::block_sumsq<WM * WN * 64>(sq, s_w, f.sumsq + slot);
}

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K>
int launch(hipStream_t st, const GemmParams& p, int splits) {
  constexpr int NBUF = WM * WN == 4 ? 2 : 3;
  dim3 grid(ppo::ceil_div(p.N, BN), ppo::ceil_div(p.M, BM), splits * p.towers);
  hipLaunchKernelGGL((gemm_f32d_kernel<BM, BN, WM, WN, A_K, B_K, NBUF>), grid, dim3(WM * WN * 64), 0, st, p);
  return ppo::check_launch("ppo_gemm_f32");
}

template <bool A_K, bool B_K>
int launch_tile(hipStream_t st, const GemmParams& p, int splits, int tile) {
  switch (tile) {
    case 0: return launch<128, 128, 2, 2, A_K, B_K>(st, p, splits);
    case 1: return launch<128, 64, 2, 2, A_K, B_K>(st, p, splits);
    case 2: return launch<64, 128, 2, 2, A_K, B_K>(st, p, splits);
    case 8: return launch<128, 256, 2, 4, A_K, B_K>(st, p, splits);
    case 9: return launch<256, 128, 4, 2, A_K, B_K>(st, p, splits);
    default: return launch<64, 64, 2, 2, A_K, B_K>(st, p, splits);
  }
}

}  // namespace

// The weight-gradient group (A k-outer, B k-outer) on 64 x 64 tiles.
int launch_dw_group(hipStream_t st, const F32Group& g) {
  const int total = g.start[g.count];
  hipLaunchKernelGGL((gemm_f32d_group_kernel<64, 64, 2, 2, false, false, 2>), dim3(total), dim3(256), 0, st, g);
  return ppo::check_launch("ppo_gemm_f32_dw_group");
}

bool final_parts_supported(int splits) {
  if (splits == 32 || splits == 64) return true;   // two-level sums
  switch (splits) {
#define PPO_F32_FINAL_CASE(S) \
  case S:
    PPO_F32_FINAL_PARTS(PPO_F32_FINAL_CASE)
#undef PPO_F32_FINAL_CASE
    return true;
    default: return false;
  }
}

int launch_dw_group_final(hipStream_t st, const F32Group& g, const ppo_gr::DwFinal& f) {
  const int total = g.start[g.count] + f.rpad;
  hipLaunchKernelGGL((gemm_f32d_group_final_kernel<64, 64, 2, 2, 2, F32D_FINAL_KIDX>), dim3(total), dim3(256), 0, st,
                     g, f);
  return ppo::check_launch("ppo_gemm_f32_dw_group_final");
}

int launch_dma(hipStream_t st, const GemmParams& p, int splits, int tile, int a_layout, int b_layout) {
  if (a_layout == 0 && b_layout == 0) return launch_tile<true, false>(st, p, splits, tile);
  if (a_layout == 0 && b_layout == 1) return launch_tile<true, true>(st, p, splits, tile);
  if (a_layout == 1 && b_layout == 0) return launch_tile<false, false>(st, p, splits, tile);
  return launch_tile<false, true>(st, p, splits, tile);
}

}  // namespace ppo_f32
