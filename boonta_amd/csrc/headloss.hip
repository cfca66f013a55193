// Fused policy/value heads + PPO loss + head backward over one minibatch.
//
// Follows loss_fn of boonta/algorithms/ppo.py:77-146 (recurrent_ppo.py:101-184)
// with the heads of boonta/networks/heads.py:9-45 (a Dense layer each, or one
// Dense feeding both when actor and critic share the torso) and the
// distributions of boonta/networks/distributions.py:8-57.
//
// One workgroup of 4 wave64s owns a tile of 64 minibatch rows and does the
// head algebra on matrix cores (v_mfma_f32_16x16x4f32), with every operand
// loaded in one pass so the global-load latency is paid a few times per tile
// rather than once per row:
//   A. head outputs OUT[64, 16] = H[64, F] Wa[F, 16] (each wave 16 rows; the
//      value of separate towers is one more column from Hc wc) -> LDS;
//   B. one lane per row: the loss, its statistics and the cotangents of the
//      head outputs (jax's tie rules for min / max / clip) -> LDS, with the
//      block's statistic, bias and Gaussian-scale partials;
//   C. per 16-feature block (dealt round-robin to the waves) over the tile's
//      64 rows: C1, the cotangent of each head input, dH = dOUT Wa^T times the
//      derivative of the torso's last activation, and C2, the head weight
//      gradient partial H^T dOUT, sharing one load of the H block.
// Every loop issues the loads of four 16-wide steps before their MFMAs, so
// four global round trips overlap.
// Per-block partials are summed in a fixed order by the gradient reduce, so
// results do not depend on scheduling.  F must be a multiple of 16 (<= 512)
// and the heads have at most 16 outputs.
#include "headloss.h"

#include <algorithm>
#include <type_traits>

using namespace ppo_hl;

namespace {

template <bool SEP, int ACT>
__global__ void __launch_bounds__(HL_THREADS) head_loss_kernel(HeadLossParams p) {
  __shared__ __attribute__((aligned(16))) float s_out[1][TR][LDO];
  __shared__ __attribute__((aligned(16))) float s_dout[TR][LDO];
  __shared__ double s_st[TR][NSTAT];
  __shared__ float s_dsc[TR][16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;   // MFMA row (A) / column (B, D)
  const int kq = lane >> 4;   // MFMA k group; D rows 4 * kq + v
  const int F = p.F;
  const int r0 = blockIdx.x * TR;
  const int64_t blk = blockIdx.x;

  // phase B's inputs, loaded first
  LaneIn lin[TR / 16];
  lane_samples(p, r0, threadIdx.x, lin);
  lane_gathers(p, threadIdx.x & 15, lin);
  const ColConst cc = load_cols(p, SEP, threadIdx.x & 15);

  // ---------------- A. head outputs of the wave's 16 rows
  {
    const int row = r0 + 16 * wave + li;
    const bool live = row < p.rows;
    const float* hrow = p.ha + (int64_t)(live ? row : 0) * p.ldha;
    const float* crow = SEP ? p.hc + (int64_t)(live ? row : 0) * p.ldhc : nullptr;
    const bool jv = li < p.na;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f}, accc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < F; k0 += 64) {
      floatx4 av[4], cv[4];
      float bv[4][4], wv[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int k = k0 + 16 * u + 4 * kq;
        const bool in = live && k0 + 16 * u < F;
        av[u] = in ? *reinterpret_cast<const floatx4*>(hrow + k) : floatx4{0.f, 0.f, 0.f, 0.f};
        if (SEP) cv[u] = in ? *reinterpret_cast<const floatx4*>(crow + k) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bool kin = k0 + 16 * u < F;
          bv[u][s] = (jv && kin) ? p.wa[(int64_t)(k + s) * p.ldwa + li] : 0.f;
          if (SEP) wv[u][s] = (li == 0 && kin) ? p.wc[(int64_t)(k + s) * p.ldwc] : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc = mfma4(av[u], bv[u], acc);
        if (SEP) accc = mfma4(cv[u], wv[u], accc);
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      s_out[0][16 * wave + 4 * kq + v][li] = acc[v];
      if (SEP && li == 0) s_out[0][16 * wave + 4 * kq + v][16] = accc[v];
    }
  }
  __syncthreads();

  // ---------------- B. loss and output cotangents (element-parallel)
  phase_b<TR, 1, SEP>(p, blk, s_out, s_dout, s_st, s_dsc, lin, cc);

  // ---------------- C. per 16-feature block (blocks dealt round-robin to the
  // waves), over all the tile's rows: C2, the head weight gradient partial
  // H^T dOUT, and C1, the cotangent of the head inputs dOUT W^T times the
  // torso activation's derivative.  One load of H[rows, block] serves both:
  // C2's operand, and C1's activation input when that is the head input
  // itself (relu / tanh outputs), so H is read twice per launch, not three
  // times.
  {
    const bool a_is_h = p.aux_a == p.ha && p.ldaux_a == p.ldha;
    const bool c_is_h = SEP && p.aux_c == p.hc && p.ldaux_c == p.ldhc;
    for (int fb = 16 * wave; fb < F; fb += 64) {
      const int f = fb + li;  // C2: A row = feature; C1: B / D column = feature
      floatx4 av[TR / 16], cv[TR / 16];
#pragma unroll
      for (int cc = 0; cc < TR / 16; ++cc) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int row = r0 + 16 * cc + 4 * kq + s;
          const bool ok = row < p.rows;
          av[cc][s] = ok ? p.ha[(int64_t)row * p.ldha + f] : 0.f;
          cv[cc][s] = (SEP && ok) ? p.hc[(int64_t)row * p.ldhc + f] : 0.f;
        }
      }
      float wb[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int j = 4 * kq + s;
        wb[s] = j < p.na ? p.wa[(int64_t)f * p.ldwa + j] : 0.f;
      }
      const float wcf = SEP ? p.wc[(int64_t)f * p.ldwc] : 0.f;
      floatx4 acc = {0.f, 0.f, 0.f, 0.f}, accc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < TR / 16; ++cc) {
        float bv[4], wv[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int rr = 16 * cc + 4 * kq + s;
          bv[s] = s_dout[rr][li];
          wv[s] = (SEP && li == 0) ? s_dout[rr][16] : 0.f;
        }
        acc = mfma4(av[cc], bv, acc);
        if (SEP) accc = mfma4(cv[cc], wv, accc);
        // C1 for rows 16 cc + 4 kq + v of this feature block
        const bool live = r0 + 16 * cc + li < p.rows;
        const floatx4 dv4 = *reinterpret_cast<const floatx4*>(&s_dout[16 * cc + li][4 * kq]);
        const floatx4 a_in = live ? dv4 : floatx4{0.f, 0.f, 0.f, 0.f};
        const floatx4 g = mfma4(a_in, wb, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int rr = 16 * cc + 4 * kq + v;
          const int row = r0 + rr;
          if (row >= p.rows) continue;
          float d = g[v];
          if (has_act<ACT>(p.act_a))
            d *= dact<ACT>(p.act_a, a_is_h ? av[cc][v] : p.aux_a[(int64_t)row * p.ldaux_a + f]);
          p.dha[(int64_t)row * p.lddha + f] = d;
          if (SEP) {
            float dc = s_dout[rr][16] * wcf;
            if (has_act<ACT>(p.act_c))
              dc *= dact<ACT>(p.act_c, c_is_h ? cv[cc][v] : p.aux_c[(int64_t)row * p.ldaux_c + f]);
            p.dhc[(int64_t)row * p.lddhc + f] = dc;
          }
        }
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int ff = fb + 4 * kq + v;
        if (li < (int)p.ldwa) p.wpart_a[(blk * F + ff) * p.ldwa + li] = acc[v];
        if (SEP && li < (int)p.ldwc) p.wpart_c[(blk * F + ff) * p.ldwc + li] = li == 0 ? accc[v] : 0.f;
      }
    }
  }
}

// The same computation for small minibatches: a workgroup owns TS = 16 rows
// and its four waves split the features instead of the rows (16-feature
// blocks fb = 16 (wave + 4 i), i < NB), so a minibatch of a few thousand
// rows still spreads over hundreds of workgroups.  Every operand of phases
// A, C1 and C2 (none depends on the loss) and the rows' rollout inputs are
// loaded before the first MFMA: one global round trip per phase chain.
// Phase A's four per-wave partial head outputs are summed in wave order.
constexpr int TS = 16;

template <bool SEP, int NB, int ACT>
__global__ void __launch_bounds__(HL_THREADS) head_loss_fs_kernel(HeadLossParams p) {
  __shared__ __attribute__((aligned(16))) float s_part[4][TS][LDO];
  __shared__ __attribute__((aligned(16))) float s_dout[TS][LDO];
  __shared__ double s_st[TS][NSTAT];
  __shared__ float s_dsc[TS][16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int kq = lane >> 4;
  const int F = p.F;
  const int r0 = blockIdx.x * TS;  // < rows: the grid has ceil(rows / TS) blocks
  const int64_t blk = blockIdx.x;
  const int last = p.rows - 1;

  // phase B's sample indices (thread: row threadIdx.x / 16, column
  // threadIdx.x % 16); their gathers follow the operand loads below
  LaneIn lin[1];
  lane_samples(p, r0, threadIdx.x, lin);
  const ColConst cc = load_cols(p, SEP, threadIdx.x & 15);

  // ---- loads of phases A, C1, C2 (clamped in-range addresses, zeroed after)
  // A: lane (row li, k group kq); C1 / C2: lane (feature li, rows 4 kq + s)
  const bool liveA = r0 + li < p.rows;
  const int64_t rowA = min(r0 + li, last);
  int64_t rowq[4];
  bool liveq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    liveq[q] = r0 + 4 * kq + q < p.rows;
    rowq[q] = min(r0 + 4 * kq + q, last);
  }
  const int ja = min(li, (int)p.ldwa - 1);  // head output column of A's B operand
  floatx4 hA[NB], cA[NB];
  float wA[NB][4], wC[NB][4], bT[NB][4], xa[NB][4], xc[NB][4], h2[NB][4], c2[NB][4], wcf[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int fb = 16 * (wave + 4 * i);
    const int fbc = fb < F ? fb : 0;
    hA[i] = *reinterpret_cast<const floatx4*>(p.ha + rowA * p.ldha + fbc + 4 * kq);
    if (SEP) cA[i] = *reinterpret_cast<const floatx4*>(p.hc + rowA * p.ldhc + fbc + 4 * kq);
    const int f = fbc + li;
    if (SEP) wcf[i] = p.wc[(int64_t)f * p.ldwc];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      wA[i][q] = p.wa[(int64_t)(fbc + 4 * kq + q) * p.ldwa + ja];
      if (SEP) wC[i][q] = p.wc[(int64_t)(fbc + 4 * kq + q) * p.ldwc];
      bT[i][q] = p.wa[(int64_t)f * p.ldwa + min(4 * kq + q, (int)p.ldwa - 1)];
      if (p.act_a != ACT_NONE) xa[i][q] = p.aux_a[rowq[q] * p.ldaux_a + f];
      if (SEP && p.act_c != ACT_NONE) xc[i][q] = p.aux_c[rowq[q] * p.ldaux_c + f];
      h2[i][q] = p.ha[rowq[q] * p.ldha + f];
      if (SEP) c2[i][q] = p.hc[rowq[q] * p.ldhc + f];
    }
  }
  lane_gathers(p, threadIdx.x & 15, lin);
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const bool fin = 16 * (wave + 4 * i) < F;
    const floatx4 z4 = {0.f, 0.f, 0.f, 0.f};
    hA[i] = (fin && liveA) ? hA[i] : z4;
    if (SEP) cA[i] = (fin && liveA) ? cA[i] : z4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      wA[i][q] = (fin && li < p.na) ? wA[i][q] : 0.f;
      if (SEP) wC[i][q] = (fin && li == 0) ? wC[i][q] : 0.f;
      bT[i][q] = (fin && 4 * kq + q < p.na) ? bT[i][q] : 0.f;
      h2[i][q] = (fin && liveq[q]) ? h2[i][q] : 0.f;
      if (SEP) c2[i][q] = (fin && liveq[q]) ? c2[i][q] : 0.f;
    }
  }

  // ---------------- A. per-wave partial head outputs of the 16 rows
  {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f}, accc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      acc = mfma4(hA[i], wA[i], acc);
      if (SEP) accc = mfma4(cA[i], wC[i], accc);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      s_part[wave][4 * kq + v][li] = acc[v];
      if (SEP && li == 0) s_part[wave][4 * kq + v][16] = accc[v];
    }
  }
  __syncthreads();

  // ---------------- B. loss and output cotangents (element-parallel)
  phase_b<TS, 4, SEP>(p, blk, s_part, s_dout, s_st, s_dsc, lin, cc);

  // ---------------- C1. cotangent of the head inputs; C2. head weight gradient partial
  const floatx4 dv4 = *reinterpret_cast<const floatx4*>(&s_dout[li][4 * kq]);
  const floatx4 a_in = liveA ? dv4 : floatx4{0.f, 0.f, 0.f, 0.f};
  float dq[4], dvq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    dq[q] = s_dout[4 * kq + q][li];
    dvq[q] = s_dout[4 * kq + q][16];
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int fb = 16 * (wave + 4 * i);
    if (fb >= F) break;
    const int f = fb + li;
    const floatx4 g = mfma4(a_in, bT[i], floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (!liveq[v]) continue;
      const int64_t row = rowq[v];
      float d = g[v];
      if (has_act<ACT>(p.act_a)) d *= dact<ACT>(p.act_a, xa[i][v]);
      p.dha[row * p.lddha + f] = d;
      if (SEP) {
        float dc = dvq[v] * wcf[i];
        if (has_act<ACT>(p.act_c)) dc *= dact<ACT>(p.act_c, xc[i][v]);
        p.dhc[row * p.lddhc + f] = dc;
      }
    }
    float wv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) wv[q] = li == 0 ? dvq[q] : 0.f;
    const floatx4 gw = mfma4(floatx4{h2[i][0], h2[i][1], h2[i][2], h2[i][3]}, dq, floatx4{0.f, 0.f, 0.f, 0.f});
    floatx4 gc = {0.f, 0.f, 0.f, 0.f};
    if (SEP) gc = mfma4(floatx4{c2[i][0], c2[i][1], c2[i][2], c2[i][3]}, wv, gc);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int ff = fb + 4 * kq + v;
      if (li < (int)p.ldwa) p.wpart_a[(blk * F + ff) * p.ldwa + li] = gw[v];
      if (SEP && li < (int)p.ldwc) p.wpart_c[(blk * F + ff) * p.ldwc + li] = li == 0 ? gc[v] : 0.f;
    }
  }
}

// Shared heads (one Dense over the torso output feeding every head output),
// large minibatches: the head input tile is read from HBM once and kept in
// registers for all three phases.  A workgroup owns 64 rows; wave w owns the
// 64 features [64 w, 64 w + 64) of all of them, lane (li, kq) holding
// H[16 cc + 4 kq + s][64 w + 4 li + m] (cc, s, m < 4) as sixteen float4.
// That layout serves C1 and C2 on MFMA directly (their 16-feature MFMA
// columns are the features 64 w + 4 li + m of one m, their row index is
// 4 kq + s); phase A, which contracts over the features, forms each lane's
// partial products over its four features and sums the sixteen lanes of a
// row group by a reduce-scatter of xor shuffles (each level keeps half of
// the values), then the four waves' partials meet in LDS and phase B sums
// them in wave order.  F <= 256, a multiple of 16.
constexpr int RT_F = 256;

// One level of the reduce-scatter over a row of 16 lanes: a lane keeps the
// half of its first n values selected by its lane bit M and adds the other
// half of lane (l xor M).  The halves are chosen with bit masks, not a
// select, which the compiler would turn into a lane-dependent index into
// the register array.
template <int M, int n, int N>
__device__ __forceinline__ void rs_level(float (&v)[N], int li) {
  const uint32_t hi = (li & M) ? 0xffffffffu : 0u;
#pragma unroll
  for (int k = 0; k < n / 2; ++k) {
    const uint32_t lo_b = __float_as_uint(v[k]), hi_b = __float_as_uint(v[n / 2 + k]);
    const float keep = __uint_as_float((hi_b & hi) | (lo_b & ~hi));
    const float send = __uint_as_float((lo_b & hi) | (hi_b & ~hi));
    v[k] = keep + ppo::xor16<M>(send);
  }
}

// Sums each of the 4 JP values over the 16 lanes of a row, scattered: lane
// li ends with the sums of values [li * JP / 4, (li + 1) * JP / 4) in
// v[0 .. JP / 4).
template <int JP>
__device__ __forceinline__ void reduce_scatter16(float (&v)[4 * JP], int li) {
  constexpr int N = 4 * JP;
  rs_level<8, N>(v, li);
  rs_level<4, N / 2>(v, li);
  rs_level<2, N / 4>(v, li);
  rs_level<1, N / 8>(v, li);
}

template <int JP, bool AUX, int ACT>
__global__ void __launch_bounds__(HL_THREADS) head_loss_rt_kernel(HeadLossParams p) {
  __shared__ __attribute__((aligned(16))) float s_part[4][TR][LDO];
  __shared__ __attribute__((aligned(16))) float s_dout[TR][LDO];
  __shared__ double s_st[TR][NSTAT];
  __shared__ float s_dsc[TR][16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int kq = lane >> 4;
  const int F = p.F;
  const int r0 = blockIdx.x * TR;
  const int64_t blk = blockIdx.x;
  const int last = p.rows - 1;
  const int f0 = 64 * wave + 4 * li;  // this lane's four features f0 + m
  const bool fin = f0 < F;             // F % 16 == 0: all four or none

  // ---- every load first: phase B's sample indices, the head input (and
  // activation input) tile, the lane's head kernel rows, then the rollout
  // gathers that need the indices
  constexpr int RW = JP <= 8 ? 8 : 16;   // phase B's lanes per row
  LaneIn lin[TR * RW / HL_THREADS];
  lane_samples<TR * RW / HL_THREADS, RW>(p, r0, threadIdx.x, lin);
  floatx4 h[4][4], xa[AUX ? 4 : 1][4];
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = r0 + 16 * cc + 4 * kq + q;
      const int64_t rc = min(r, last);
      const int fc = fin ? f0 : 0;
      h[cc][q] = *reinterpret_cast<const floatx4*>(p.ha + rc * p.ldha + fc);
      if (AUX) xa[cc][q] = *reinterpret_cast<const floatx4*>(p.aux_a + rc * p.ldaux_a + fc);
    }
  }
  // wA[m][j] = W[f0 + m][j] (phase A), 16-byte loads (ldwa is a multiple of
  // 4, <= JP)
  float wA[4][JP];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float* wrow = p.wa + (int64_t)(fin ? f0 + m : 0) * p.ldwa;
#pragma unroll
    for (int j4 = 0; j4 < JP / 4; ++j4) {
      const floatx4 w4 = *reinterpret_cast<const floatx4*>(wrow + min(4 * j4, (int)p.ldwa - 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) wA[m][4 * j4 + e] = w4[e];
    }
  }
  lane_gathers(p, threadIdx.x % RW, lin);
  const ColConst cc0 = load_cols(p, false, threadIdx.x % RW);
  // zero what lies outside the rows, the features or the head outputs
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool ok = fin && r0 + 16 * cc + 4 * kq + q < p.rows;
      h[cc][q] = ok ? h[cc][q] : floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int j = 0; j < JP; ++j) wA[m][j] = (fin && j < p.na) ? wA[m][j] : 0.f;
  }
  // C1's B operand for k step s: wb[m][s] = W[f0 + m][kq + 4 s], taken from
  // wA by bit masks on kq (a select would become a lane-dependent index)
  constexpr int SJ = JP / 4;
  float wb[4][SJ];
  {
    uint32_t sel[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) sel[c] = kq == c ? 0xffffffffu : 0u;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int s2 = 0; s2 < SJ; ++s2) {
        uint32_t b = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) b |= __float_as_uint(wA[m][4 * s2 + c]) & sel[c];
        wb[m][s2] = __uint_as_float(b);
      }
    }
  }

  // ---------------- A. head outputs: per-lane products over the lane's four
  // features, summed over the sixteen lanes of each row group, per wave
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    float v[4 * JP];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int j = 0; j < JP; ++j) {
        float a = h[cc][q][0] * wA[0][j];
        a = __fmaf_rn(h[cc][q][1], wA[1][j], a);
        a = __fmaf_rn(h[cc][q][2], wA[2][j], a);
        v[q * JP + j] = __fmaf_rn(h[cc][q][3], wA[3][j], a);
      }
    }
    reduce_scatter16<JP>(v, li);
    // lane li now holds row 4 kq + (li >> 2) of this group, outputs
    // (li & 3) * JP / 4 + c
    const int rr = 16 * cc + 4 * kq + (li >> 2);
#pragma unroll
    for (int c = 0; c < JP / 4; ++c) s_part[wave][rr][(li & 3) * (JP / 4) + c] = v[c];
  }
  __syncthreads();

  // ---------------- B. loss and output cotangents (element-parallel)
  phase_b<TR, 4, false, RW>(p, blk, s_part, s_dout, s_st, s_dsc, lin, cc0);

  // ---------------- C1. input cotangent dH = dOUT W^T (times the activation's
  // derivative) of every row group, from the same registers
  // (k step s contracts head outputs kq + 4 s: SJ = JP / 4 steps cover them)
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    const bool liveA = r0 + 16 * cc + li < p.rows;
    float a_in[SJ];
#pragma unroll
    for (int s2 = 0; s2 < SJ; ++s2) a_in[s2] = liveA ? s_dout[16 * cc + li][kq + 4 * s2] : 0.f;
    floatx4 g[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      g[m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < SJ; ++s2) g[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(a_in[s2], wb[m][s2], g[m], 0, 0, 0);
    }
    // g[m][v]: row 16 cc + 4 kq + v, feature f0 + m
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = r0 + 16 * cc + 4 * kq + v;
      if (!fin || r >= p.rows) continue;
      floatx4 d = {g[0][v], g[1][v], g[2][v], g[3][v]};
      if (has_act<ACT>(p.act_a)) {
        const floatx4 x = AUX ? xa[cc][v] : h[cc][v];
#pragma unroll
        for (int m = 0; m < 4; ++m) d[m] *= dact<ACT>(p.act_a, x[m]);
      }
      *reinterpret_cast<floatx4*>(p.dha + (int64_t)r * p.lddha + f0) = d;
    }
  }

  // ---------------- C2. head weight gradient partial H^T dOUT over the 64 rows
  float dq[4][4];
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
#pragma unroll
    for (int q = 0; q < 4; ++q) dq[cc][q] = s_dout[16 * cc + 4 * kq + q][li];
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const floatx4 a = {h[cc][0][m], h[cc][1][m], h[cc][2][m], h[cc][3][m]};
      acc = mfma4(a, dq[cc], acc);
    }
    // acc[v]: feature 64 w + 4 (4 kq + v) + m, output li
    if (li < (int)p.ldwa) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int f = 64 * wave + 4 * (4 * kq + v) + m;
        if (f < F) p.wpart_a[(blk * F + f) * p.ldwa + li] = acc[v];
      }
    }
  }
}

}  // namespace

#ifndef PPO_HL_SMALL_ROWS
#define PPO_HL_SMALL_ROWS 16384  // minibatches up to this many rows take the feature-split kernel
#endif

// Blocks the fused kernel launches for `rows` (the partial buffers' leading
// extent): one per 16-row tile up to PPO_HL_SMALL_ROWS rows, else one per
// 64-row tile.
PPO_EXPORT int ppo_head_loss_blocks(int rows) {
  return std::max(1, ppo::ceil_div(rows, rows <= PPO_HL_SMALL_ROWS ? TS : TR));
}

// Largest head width (outputs of group a) and feature width the fused kernel
// takes; the feature width must also be a multiple of 16.
PPO_EXPORT int ppo_head_loss_max_outputs(void) { return 16; }
PPO_EXPORT int ppo_head_loss_max_features(void) { return 512; }

int ppo_hl::head_loss_setup(
    HeadLossParams& p, const char* name, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha,
    const float* wa, int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc,
    int64_t ldwc, const float* bc, int F, int A, const float* scale_param, const int32_t* action_i,
    const float* action_f, const float* old_logp, const float* old_value, const float* adv, const float* ret,
    int act_a, const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature, float* ratio_out, int ratio_envs, int ratio_steps, int64_t sample_stride) {
  const bool sep = hc != nullptr;
  if (sample_stride < 1) return ppo::set_error(PPO_ERR_ARG, "%s: sample_stride must be at least 1", name);
  if (rows < 0 || F <= 0 || F > 512 || F % 16 != 0 || na <= 0 || na > 16 || ldwa < na || ldwa > 16 || A <= 0 ||
      A > 16 ||
      (dist != DIST_CATEGORICAL && dist != DIST_GAUSSIAN) || !ha || !wa || !ba || !old_logp || !old_value ||
      !adv || !ret || !dha || !wpart_a || !bpart_a || !stats_partial || temperature <= 0.f)
    return ppo::set_error(PPO_ERR_ARG, "%s: bad argument (rows=%d F=%d na=%d A=%d)", name, rows, F, na, A);
  if (sep && (!wc || !bc || !dhc || !wpart_c || !bpart_c || ldwc < 1))
    return ppo::set_error(PPO_ERR_ARG, "%s: separate heads need the critic buffers", name);
  if ((dist == DIST_CATEGORICAL && !action_i) || (dist == DIST_GAUSSIAN && !action_f))
    return ppo::set_error(PPO_ERR_ARG, "%s: missing actions", name);
  if (scale_param && !dscale_partial) return ppo::set_error(PPO_ERR_ARG, "%s: missing dscale buffer", name);
  if ((act_a != ACT_NONE && !aux_a) || (sep && act_c != ACT_NONE && !aux_c))
    return ppo::set_error(PPO_ERR_ARG, "%s: activation derivative needs aux", name);
  if (sep && ldwc > 16) return ppo::set_error(PPO_ERR_ARG, "%s: ldwc > 16", name);
  if ((reinterpret_cast<uintptr_t>(ha) & 15) || ldha % 4 || (sep && ((reinterpret_cast<uintptr_t>(hc) & 15) || ldhc % 4)))
    return ppo::set_error(PPO_ERR_ARG, "%s: head inputs need 16-byte aligned rows", name);
  p = HeadLossParams{};
  p.dist = dist; p.rows = rows; p.idx = idx;
  p.ha = ha; p.ldha = ldha; p.wa = wa; p.ldwa = ldwa; p.ba = ba; p.na = na;
  p.hc = hc; p.ldhc = ldhc; p.wc = wc; p.ldwc = ldwc; p.bc = bc;
  p.F = F; p.A = A; p.scale_param = scale_param; p.action_i = action_i; p.action_f = action_f;
  p.old_logp = old_logp; p.old_value = old_value; p.adv = adv; p.ret = ret;
  p.act_a = act_a; p.aux_a = aux_a; p.ldaux_a = ldaux_a; p.dha = dha; p.lddha = lddha;
  p.act_c = act_c; p.aux_c = aux_c; p.ldaux_c = ldaux_c; p.dhc = dhc; p.lddhc = lddhc;
  p.wpart_a = wpart_a; p.bpart_a = bpart_a; p.wpart_c = wpart_c; p.bpart_c = bpart_c;
  p.dscale_partial = dscale_partial; p.stats_partial = stats_partial;
  p.clip_eps = clip_eps; p.clip_value_loss = clip_value_loss; p.ent_coef = ent_coef; p.vf_coef = vf_coef;
  p.inv_n = rows > 0 ? 1.f / (float)rows : 0.f; p.temperature = temperature;
  p.ratio_out = ratio_out; p.ratio_envs = ratio_envs; p.ratio_steps = ratio_steps;
  p.sample_stride = sample_stride;
  p.rec4 = sample_stride % 4 == 0 && !(reinterpret_cast<uintptr_t>(old_logp) & 15) && old_value == old_logp + 1 &&
           adv == old_logp + 2 && ret == old_logp + 3;
  return PPO_OK;
}

static int head_loss_impl(
    void* stream, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha, const float* wa,
    int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc, int64_t ldwc,
    const float* bc, int F, int A, const float* scale_param, const int32_t* action_i, const float* action_f,
    const float* old_logp, const float* old_value, const float* adv, const float* ret, int act_a,
    const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature, float* ratio_out, int ratio_envs, int ratio_steps, int64_t sample_stride) {
  const bool sep = hc != nullptr;
  HeadLossParams p;
  const int rc = head_loss_setup(p, "ppo_head_loss_f32", dist, rows, idx, ha, ldha, wa, ldwa, ba, na, hc, ldhc, wc,
                                 ldwc, bc, F, A, scale_param, action_i, action_f, old_logp, old_value, adv, ret,
                                 act_a, aux_a, ldaux_a, dha, lddha, act_c, aux_c, ldaux_c, dhc, lddhc, wpart_a,
                                 bpart_a, wpart_c, bpart_c, dscale_partial, stats_partial, clip_eps, clip_value_loss,
                                 ent_coef, vf_coef, temperature, ratio_out, ratio_envs, ratio_steps, sample_stride);
  if (rc != PPO_OK) return rc;
  if (rows == 0) return PPO_OK;
  const int blocks = ppo_head_loss_blocks(rows);
  hipStream_t st = ppo::as_stream(stream);
  // the activation as a template constant when both towers use one of
  // none / relu / silu (else the run-time switch, -1)
  const int actc = (!sep || act_a == act_c) && (act_a == ACT_NONE || act_a == ACT_RELU || act_a == ACT_SILU) ? act_a
                                                                                                              : -1;
  auto launch = [&](auto sep_c, auto act_c_) {
    constexpr bool S = decltype(sep_c)::value;
    constexpr int AC = decltype(act_c_)::value;
    if (rows <= PPO_HL_SMALL_ROWS) {
      const int nb = ppo::ceil_div(F, 64);  // 16-feature blocks per wave
      if (nb <= 1) hipLaunchKernelGGL((head_loss_fs_kernel<S, 1, AC>), dim3(blocks), dim3(HL_THREADS), 0, st, p);
      else if (nb <= 2) hipLaunchKernelGGL((head_loss_fs_kernel<S, 2, AC>), dim3(blocks), dim3(HL_THREADS), 0, st, p);
      else if (nb <= 4) hipLaunchKernelGGL((head_loss_fs_kernel<S, 4, AC>), dim3(blocks), dim3(HL_THREADS), 0, st, p);
      else hipLaunchKernelGGL((head_loss_fs_kernel<S, 8, AC>), dim3(blocks), dim3(HL_THREADS), 0, st, p);
    } else if (!S && F <= RT_F && ldwa % 4 == 0 && (reinterpret_cast<uintptr_t>(wa) & 15) == 0) {
      // the shared head's input read once, kept in registers
      const bool aux = act_a != ACT_NONE && !(aux_a == ha && ldaux_a == ldha);
      const int jp = ldwa <= 4 ? 4 : ldwa <= 8 ? 8 : 16;
      auto rt = [&](auto jp_c, auto aux_c) {
        hipLaunchKernelGGL((head_loss_rt_kernel<decltype(jp_c)::value, decltype(aux_c)::value, AC>), dim3(blocks),
                           dim3(HL_THREADS), 0, st, p);
      };
      auto by_jp = [&](auto aux_c) {
        if (jp == 4) rt(std::integral_constant<int, 4>{}, aux_c);
        else if (jp == 8) rt(std::integral_constant<int, 8>{}, aux_c);
        else rt(std::integral_constant<int, 16>{}, aux_c);
      };
      if (aux) by_jp(std::true_type{});
      else by_jp(std::false_type{});
    } else {
      hipLaunchKernelGGL((head_loss_kernel<S, AC>), dim3(blocks), dim3(HL_THREADS), 0, st, p);
    }
  };
  auto by_act = [&](auto sep_c) {
    switch (actc) {
      case ACT_NONE: launch(sep_c, std::integral_constant<int, ACT_NONE>{}); break;
      case ACT_RELU: launch(sep_c, std::integral_constant<int, ACT_RELU>{}); break;
      case ACT_SILU: launch(sep_c, std::integral_constant<int, ACT_SILU>{}); break;
      default: launch(sep_c, std::integral_constant<int, -1>{}); break;
    }
  };
  if (sep) by_act(std::true_type{});
  else by_act(std::false_type{});
  return ppo::check_launch("ppo_head_loss_f32");
}

PPO_EXPORT int ppo_head_loss_f32(
    void* stream, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha, const float* wa,
    int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc, int64_t ldwc,
    const float* bc, int F, int A, const float* scale_param, const int32_t* action_i, const float* action_f,
    const float* old_logp, const float* old_value, const float* adv, const float* ret, int act_a,
    const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature, int64_t sample_stride) {
  return head_loss_impl(stream, dist, rows, idx, ha, ldha, wa, ldwa, ba, na, hc, ldhc, wc, ldwc, bc, F, A,
                        scale_param, action_i, action_f, old_logp, old_value, adv, ret, act_a, aux_a, ldaux_a, dha,
                        lddha, act_c, aux_c, ldaux_c, dhc, lddhc, wpart_a, bpart_a, wpart_c, bpart_c, dscale_partial,
                        stats_partial, clip_eps, clip_value_loss, ent_coef, vf_coef, temperature, nullptr, 1, 1,
                        sample_stride);
}

// ppo_head_loss_f32 that also writes each row's ratio exp(logp - old_logp)
// into ratio_out[(s % envs) * steps + s / envs], s = idx[row] = t * envs + env
// (RecurrentPuPO keeps the last ratio of every env and step).  Every sample
// index must be below envs * steps.
PPO_EXPORT int ppo_head_loss_ratio_f32(
    void* stream, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha, const float* wa,
    int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc, int64_t ldwc,
    const float* bc, int F, int A, const float* scale_param, const int32_t* action_i, const float* action_f,
    const float* old_logp, const float* old_value, const float* adv, const float* ret, int act_a,
    const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature, float* ratio_out, int envs, int steps, int64_t sample_stride) {
  if (!ratio_out || envs < 1 || steps < 1 || (int64_t)envs * steps > INT32_MAX)
    return ppo::set_error(PPO_ERR_ARG, "ppo_head_loss_ratio_f32: bad ratio buffer (envs %d, steps %d)", envs, steps);
  return head_loss_impl(stream, dist, rows, idx, ha, ldha, wa, ldwa, ba, na, hc, ldhc, wc, ldwc, bc, F, A,
                        scale_param, action_i, action_f, old_logp, old_value, adv, ret, act_a, aux_a, ldaux_a, dha,
                        lddha, act_c, aux_c, ldaux_c, dhc, lddhc, wpart_a, bpart_a, wpart_c, bpart_c, dscale_partial,
                        stats_partial, clip_eps, clip_value_loss, ent_coef, vf_coef, temperature, ratio_out, envs,
                        steps, sample_stride);
}

// One 32-byte record per sample for the fused loss's gathers, sample_stride
// 8: {old log-prob, old value, advantage, return, action (int32 bits, 0
// without), 0, 0, 0}, so that a row's four rollout scalars arrive in one
// 16-byte load and its action from the same 64-byte sector, instead of five
// scattered 4-byte reads.
__global__ void pack_samples_kernel(int64_t n, const float* __restrict__ old_logp, const float* __restrict__ old_value,
                                    const float* __restrict__ adv, const float* __restrict__ ret,
                                    const int32_t* __restrict__ action_i, float* __restrict__ rec) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const floatx4 a = {old_logp[i], old_value[i], adv[i], ret[i]};
  const floatx4 b = {action_i ? __int_as_float(action_i[i]) : 0.f, 0.f, 0.f, 0.f};
  reinterpret_cast<floatx4*>(rec)[2 * i] = a;
  reinterpret_cast<floatx4*>(rec)[2 * i + 1] = b;
}

PPO_EXPORT int ppo_pack_samples(void* stream, int64_t n, const float* old_logp, const float* old_value,
                                const float* adv, const float* ret, const int32_t* action_i, float* rec) {
  if (n < 0 || (n > 0 && (!old_logp || !old_value || !adv || !ret || !rec)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_pack_samples: bad argument (n=%lld)", (long long)n);
  if (reinterpret_cast<uintptr_t>(rec) & 15)
    return ppo::set_error(PPO_ERR_ARG, "ppo_pack_samples: records must be 16-byte aligned");
  if (n == 0) return PPO_OK;
  hipLaunchKernelGGL(pack_samples_kernel, dim3((unsigned)ppo::ceil_div64(n, 256)), dim3(256), 0,
                     ppo::as_stream(stream), n, old_logp, old_value, adv, ret, action_i, rec);
  return ppo::check_launch("ppo_pack_samples");
}
