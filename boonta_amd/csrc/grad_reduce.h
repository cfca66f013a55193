// The fixed-order sum of gradient partials shared by the gradient-assembly
// launch (adam.hip: ppo_grad_reduce) and the weight-gradient launch that
// finishes its own split-K sums (gemm_f32d.hip: ppo_gemm_f32_dw_group_final).
//
// A gradient leaf arrives as `nparts` partial buffers (split-K GEMM slices,
// per-block LayerNorm / head partials).  Its sum is always formed in the
// same association, whichever launch forms it:
//   nparts <= FEW_PARTS:       ((0 + p0) + p1) + ...          (partial order)
//   FEW_PARTS < nparts <= WIDE_PARTS: four quarters [n w / 4, n (w + 1) / 4),
//     each 0 + tree8(p_q0..q0+7) + tree8(next 8) + ... (tree8 =
//     ((a + b) + (c + d)) + ((e + f) + (g + h)), missing entries 0), then
//     ((quarter0 + quarter1) + quarter2) + quarter3
//   nparts > WIDE_PARTS:       sixteen ranges [n j / 16, n (j + 1) / 16) the
//     same way, then added in range order
// so a gradient is the same bits from either launch.
#pragma once
#include "common.h"

namespace ppo_gr {

struct Segment {
  float* dst;
  const float* src;
  int64_t count;
  int64_t part_stride;
  int nparts;
  int flags;  // SEG_ROUND_BF16: the summed gradient is rounded to bf16
};

constexpr int SEG_ROUND_BF16 = 1;

struct Chunk {
  int seg;
  int slot;  // its squared-norm partial's index in sumsq
  int64_t start;
};

constexpr int REDUCE_THREADS = 256;
constexpr int CHUNK = 256;  // elements per block: one float4 per lane of a wave
constexpr int FEW_PARTS = 4;
constexpr int WIDE_PARTS = 64;
constexpr int WIDE_CHUNK = 64;

__device__ __forceinline__ floatx4 tree8(const floatx4 (&v)[8]) {
  return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

// One block of the gradient-assembly launch (block b of its dispatch order:
// the wide chunks' blocks first, then the few-part blocks, four chunks per
// block, then the others).  part: 4 x 64 float4 of LDS.
//
// Each of the 4 waves sums a contiguous quarter of the partials for the same
// 64 float4, eight partials per step (eight loads in flight per lane; the
// last step's missing partials read a clamped partial and count as zero),
// then the quarters are added in wave order.  Few-part chunks are taken one
// per wave with all of a lane's partial loads in flight at once.  Wide
// chunks cover WIDE_CHUNK elements: lane l of wave w sums range
// j = 4 w + l / 16 for float4 l % 16, and the sixteen range sums are added
// in range order.
__device__ __forceinline__ void reduce_block(int b, const Segment* __restrict__ segs,
                                             const Chunk* __restrict__ chunks, int nchunks, int nfew, int nwide,
                                             double* __restrict__ sumsq, floatx4 (*part)[64]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int few_blocks = (nfew + 3) / 4;
  if (b < nwide) {
    const Chunk ch = chunks[nchunks - nwide + b];
    const Segment sg = segs[ch.seg];
    const int c = lane & 15, j = 4 * wave + (lane >> 4);
    const int64_t i = ch.start + 4 * c;
    const bool live = i < sg.count;
    const int q0 = (sg.nparts * j) / 16, q1 = (sg.nparts * (j + 1)) / 16;
    constexpr int U = 8;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    if (live && q1 > q0) {
      const float* src = sg.src + i;
      for (int q = q0; q < q1; q += U) {
        floatx4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int qq = min(q + u, q1 - 1);
          v[u] = *reinterpret_cast<const floatx4*>(src + (int64_t)qq * sg.part_stride);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = q + u < q1 ? v[u] : floatx4{0.f, 0.f, 0.f, 0.f};
        acc += tree8(v);
      }
    }
    part[j >> 2][16 * (j & 3) + c] = acc;  // range j of float4 c
    __syncthreads();
    if (wave == 0) {
      double sq = 0.0;
      if (lane < 16 && live) {
        floatx4 t = part[0][lane];
#pragma unroll
        for (int r = 1; r < 16; ++r) t += part[r >> 2][16 * (r & 3) + lane];
        if (sg.flags & SEG_ROUND_BF16) {
#pragma unroll
          for (int e = 0; e < 4; ++e) t[e] = ppo::bf16_round(t[e]);
        }
        *reinterpret_cast<floatx4*>(sg.dst + i) = t;
#pragma unroll
        for (int e = 0; e < 4; ++e) sq += (double)t[e] * (double)t[e];
      }
      sq = ppo::wave_sum_d(sq);
      if (lane == 0) sumsq[ch.slot] = sq;
    }
    return;
  }
  b -= nwide;
  if (b < few_blocks) {
    const int ci = 4 * b + wave;
    if (ci >= nfew) return;  // this path has no barrier
    const Chunk ch = chunks[ci];
    const Segment sg = segs[ch.seg];
    const int64_t i = ch.start + 4 * lane;
    const bool live = i < sg.count;
    floatx4 v[FEW_PARTS];
#pragma unroll
    for (int q = 0; q < FEW_PARTS; ++q)
      v[q] = (live && q < sg.nparts) ? *reinterpret_cast<const floatx4*>(sg.src + i + (int64_t)q * sg.part_stride)
                                     : floatx4{0.f, 0.f, 0.f, 0.f};
    double sq = 0.0;
    if (live) {
      floatx4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < FEW_PARTS; ++q)
        if (q < sg.nparts) t += v[q];
      if (sg.flags & SEG_ROUND_BF16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = ppo::bf16_round(t[e]);
      }
      *reinterpret_cast<floatx4*>(sg.dst + i) = t;
#pragma unroll
      for (int e = 0; e < 4; ++e) sq += (double)t[e] * (double)t[e];
    }
    sq = ppo::wave_sum_d(sq);
    if (lane == 0) sumsq[ch.slot] = sq;
    return;
  }
  const Chunk ch = chunks[nfew + (b - few_blocks)];
  const Segment sg = segs[ch.seg];
  const int64_t i = ch.start + 4 * lane;  // first element of this lane's float4
  const bool live = i < sg.count;
  const int q0 = (sg.nparts * wave) / 4, q1 = (sg.nparts * (wave + 1)) / 4;
  constexpr int U = 8;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  if (live && q1 > q0) {
    const float* s = sg.src + i;
    for (int q = q0; q < q1; q += U) {
      floatx4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int qq = min(q + u, q1 - 1);
        v[u] = *reinterpret_cast<const floatx4*>(s + (int64_t)qq * sg.part_stride);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = q + u < q1 ? v[u] : floatx4{0.f, 0.f, 0.f, 0.f};
      acc += tree8(v);
    }
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    double sq = 0.0;
    if (live) {
      floatx4 t = part[0][lane];
#pragma unroll
      for (int w = 1; w < REDUCE_THREADS / 64; ++w) t += part[w][lane];
      if (sg.flags & SEG_ROUND_BF16) {
        // the gradient of a parameter cast to bf16 arrives as a bf16 cotangent
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = ppo::bf16_round(t[e]);
      }
      *reinterpret_cast<floatx4*>(sg.dst + i) = t;
#pragma unroll
      for (int e = 0; e < 4; ++e) sq += (double)t[e] * (double)t[e];
    }
    sq = ppo::wave_sum_d(sq);
    if (lane == 0) sumsq[ch.slot] = sq;
  }
}

// The sum of S partials v[0..S) (compile-time S, at most WIDE_PARTS) in the
// association above; the reduce forms the same value for an S-part segment.
template <int S>
__device__ __forceinline__ floatx4 fixed_sum(const floatx4 (&v)[S]) {
  static_assert(S >= 1 && S <= WIDE_PARTS, "partial count out of range");
  const floatx4 z = {0.f, 0.f, 0.f, 0.f};
  if constexpr (S <= FEW_PARTS) {
    floatx4 t = z;
#pragma unroll
    for (int q = 0; q < S; ++q) t += v[q];
    return t;
  } else {
    floatx4 quarter[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int q0 = (S * w) / 4, q1 = (S * (w + 1)) / 4;
      floatx4 acc = z;
#pragma unroll
      for (int q = q0; q < q1; q += 8) {
        floatx4 g[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) g[u] = q + u < q1 ? v[q + u] : z;
        acc += tree8(g);
      }
      quarter[w] = acc;
    }
    floatx4 t = quarter[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) t += quarter[w];
    return t;
  }
}

// A weight-gradient launch that finishes its own split-K sums: the last
// split of each output tile to arrive (a per-tile arrival counter) sums the
// tile's partials in the fixed order above into the final gradient and
// writes the tile's squared-norm partial; workgroups placed before the tiles
// reduce the table's other segments.
constexpr int DW_FINAL_MAX = 8;
struct DwFinal {
  float* G[DW_FINAL_MAX];    // problem i's final gradient, [g_rows][ldg]
  int64_t ldg[DW_FINAL_MAX];
  int g_rows[DW_FINAL_MAX];  // rows of the gradient (<= M: a zero-padded input's extra rows are dropped)
  float* Gb[DW_FINAL_MAX];   // final bias gradient [N] (problems with bias partials)
  int slot0[DW_FINAL_MAX];   // problem i's first tile: its counter and sumsq index
  int splits[DW_FINAL_MAX];  // problem i's split count
  unsigned* counters;        // one per tile, then (two-level sums) eight per tile; zero between launches
  int ntiles;                // tiles of the launch (the second block of counters starts there)
  double* sumsq;
  const void* segs;          // the other segments, reduced by rblocks workgroups
  const void* chunks;
  int nchunks, nfew, nwide, rblocks, rpad;  // rpad: rblocks rounded up to a multiple of 8
  int round_bf16;            // the gradients are rounded to bf16 (bf16 layers' parameters)
};

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int SC1 = 16;  // cache policy of a device-coherent buffer access

// Largest power of two <= x (x >= 1).
constexpr int pow2_floor(int x) { return x >= 2 ? 2 * pow2_floor(x / 2) : 1; }

// The finishing sum of one BM x BN output tile (tile row tm, column tn) of
// S split partials (fp32, row pitch ldc, split stride split_stride, written
// device-coherent by other workgroups) into G (rows below rows_out, pitch
// ldg; rounded to bf16 when round_bf16), and for the first tile row the bias
// partials [S][N] (bias_part, or null) into Gb.  Thread t of NT owns float4
// t + NT i of the tile; LOADS bounds a thread's partial loads in flight.
// Returns the thread's sum of squares of the values it wrote.
template <int BM, int BN, int NT, int S, int LOADS>
__device__ __forceinline__ double finish_tile_sum(const float* C, int64_t ldc, int64_t split_stride, int rows_out,
                                                  int N, int tm, int tn, float* G, int64_t ldg, bool round_bf16,
                                                  const float* bias_part, float* Gb) {
  constexpr int POS = BM * BN / 4 / NT;
  constexpr int P0 = pow2_floor(LOADS / S > 0 ? LOADS / S : 1);
  constexpr int P = P0 < POS ? P0 : POS;
  static_assert(POS % P == 0, "positions per round must divide the tile's");
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(C), (short)0, 0x7fffffff, 0x00020000);
  const int t = threadIdx.x;
  double sq = 0.0;
  auto store = [&](float* dst, floatx4 g) {
    if (round_bf16) {
#pragma unroll
      for (int e = 0; e < 4; ++e) g[e] = ppo::bf16_round(g[e]);
    }
    *reinterpret_cast<floatx4*>(dst) = g;
#pragma unroll
    for (int e = 0; e < 4; ++e) sq += (double)g[e] * (double)g[e];
  };
#pragma unroll
  for (int i0 = 0; i0 < POS; i0 += P) {
    floatx4 v[P][S];
    bool live[P];
    int64_t dst[P];
#pragma unroll
    for (int u = 0; u < P; ++u) {
      const int e = t + NT * (i0 + u);
      const int gm = tm * BM + e / (BN / 4), gn = tn * BN + 4 * (e % (BN / 4));
      live[u] = gm < rows_out && gn < N;
      dst[u] = (int64_t)gm * ldg + gn;
      const int off = live[u] ? (int)(4 * ((int64_t)gm * ldc + gn)) : 0;
#pragma unroll
      for (int q = 0; q < S; ++q)
        v[u][q] = __builtin_bit_cast(
            floatx4, __builtin_amdgcn_raw_buffer_load_b128(rc, off + (int)(4 * q * split_stride), 0, SC1));
    }
#pragma unroll
    for (int u = 0; u < P; ++u)
      if (live[u]) store(G + dst[u], fixed_sum<S>(v[u]));
  }
  if (tm == 0 && bias_part && Gb && t < BN / 4) {
    const int gn = tn * BN + 4 * t;
    if (gn < N) {
      const __amdgpu_buffer_rsrc_t rb =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(bias_part), (short)0, 0x7fffffff, 0x00020000);
      floatx4 v[S];
#pragma unroll
      for (int q = 0; q < S; ++q)
        v[q] = __builtin_bit_cast(floatx4,
                                  __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(4 * ((int64_t)q * N + gn)), 0, SC1));
      store(Gb + gn, fixed_sum<S>(v));
    }
  }
  return sq;
}

// The first level of a two-level finishing sum (32 or 64 splits): the sum
// of splits 8 grp .. 8 grp + 7 of the tile (and of their bias partials for the
// first tile row) as tree8 — the reduce's sum of those eight partials — stored
// device-coherent over split 8 grp's partial (which no one reads after this).
template <int BM, int BN, int NT>
__device__ __forceinline__ void finish_group8(float* C, int64_t ldc, int64_t split_stride, int rows_out, int N,
                                              int tm, int tn, int grp, float* bias_part) {
  constexpr int POS = BM * BN / 4 / NT;
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, 0x7fffffff, 0x00020000);
  const int t = threadIdx.x;
  const int q0 = 8 * grp;
#pragma unroll
  for (int i = 0; i < POS; ++i) {
    const int e = t + NT * i;
    const int gm = tm * BM + e / (BN / 4), gn = tn * BN + 4 * (e % (BN / 4));
    if (gm >= rows_out || gn >= N) continue;
    const int off = (int)(4 * ((int64_t)gm * ldc + gn));
    floatx4 v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      v[q] = __builtin_bit_cast(
          floatx4, __builtin_amdgcn_raw_buffer_load_b128(rc, off + (int)(4 * (q0 + q) * split_stride), 0, SC1));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, tree8(v)), rc,
                                           off + (int)(4 * q0 * split_stride), 0, SC1);
  }
  if (tm == 0 && bias_part && t < BN / 4) {
    const int gn = tn * BN + 4 * t;
    if (gn < N) {
      const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(bias_part, (short)0, 0x7fffffff, 0x00020000);
      floatx4 v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q)
        v[q] = __builtin_bit_cast(
            floatx4, __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(4 * ((int64_t)(q0 + q) * N + gn)), 0, SC1));
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, tree8(v)), rb,
                                             (int)(4 * ((int64_t)q0 * N + gn)), 0, SC1);
    }
  }
}

// The second level for S = 8 GR splits: the GR group sums g_k (at split
// 8 k's partial) added as the reduce adds an S-part segment — quarter w is
// 0 + the tree8 sums of its eight-partial groups in order, then the quarters
// in order — into G / Gb as finish_tile_sum does.
template <int BM, int BN, int NT, int GR>
__device__ __forceinline__ double finish_level2(const float* C, int64_t ldc, int64_t split_stride, int rows_out,
                                                int N, int tm, int tn, float* G, int64_t ldg,
                                                const float* bias_part, float* Gb) {
  static_assert(GR == 4 || GR == 8, "two-level sums of 32 or 64 splits");
  constexpr int POS = BM * BN / 4 / NT;
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(C), (short)0, 0x7fffffff, 0x00020000);
  const int t = threadIdx.x;
  const floatx4 z = {0.f, 0.f, 0.f, 0.f};
  double sq = 0.0;
  auto combine = [&](const floatx4 (&g)[GR]) {
    floatx4 quarter[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      floatx4 acc = z;
#pragma unroll
      for (int k = GR * w / 4; k < GR * (w + 1) / 4; ++k) acc += g[k];
      quarter[w] = acc;
    }
    floatx4 r = quarter[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) r += quarter[w];
    return r;
  };
  auto store = [&](float* dst, floatx4 v) {
    *reinterpret_cast<floatx4*>(dst) = v;
#pragma unroll
    for (int e = 0; e < 4; ++e) sq += (double)v[e] * (double)v[e];
  };
#pragma unroll
  for (int i = 0; i < POS; ++i) {
    const int e = t + NT * i;
    const int gm = tm * BM + e / (BN / 4), gn = tn * BN + 4 * (e % (BN / 4));
    if (gm >= rows_out || gn >= N) continue;
    const int off = (int)(4 * ((int64_t)gm * ldc + gn));
    floatx4 g[GR];
#pragma unroll
    for (int k = 0; k < GR; ++k)
      g[k] = __builtin_bit_cast(floatx4,
                                __builtin_amdgcn_raw_buffer_load_b128(rc, off + (int)(4 * 8 * k * split_stride), 0, SC1));
    store(G + (int64_t)gm * ldg + gn, combine(g));
  }
  if (tm == 0 && bias_part && Gb && t < BN / 4) {
    const int gn = tn * BN + 4 * t;
    if (gn < N) {
      const __amdgpu_buffer_rsrc_t rb =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(bias_part), (short)0, 0x7fffffff, 0x00020000);
      floatx4 g[GR];
#pragma unroll
      for (int k = 0; k < GR; ++k)
        g[k] = __builtin_bit_cast(
            floatx4, __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(4 * ((int64_t)8 * k * N + gn)), 0, SC1));
      store(Gb + gn, combine(g));
    }
  }
  return sq;
}

// A workgroup's arrival at its tile once its partial stores (device-coherent)
// are complete: true for the last of the tile's splits, which then resets the
// counter.  s_last: one int of LDS.
__device__ __forceinline__ bool arrive_last(unsigned* counter, int splits, int* s_last) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned seen = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = seen + 1 == (unsigned)splits;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = last;
  }
  __syncthreads();
  return *s_last != 0;
}

// The squared-norm partial of a workgroup of NT threads (each thread's sq):
// wave sums, then the waves in order, written by thread 0.  s_w: NT / 64
// doubles of LDS.
template <int NT>
__device__ __forceinline__ void block_sumsq(double sq, double* s_w, double* out) {
  sq = ppo::wave_sum_d(sq);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = sq;
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = s_w[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) tot += s_w[w];
    *out = tot;
  }
}

}  // namespace ppo_gr
