// Whole torso chains of Dense -> LayerNorm -> activation layers (all 256
// wide, fp32) in one launch each, for the actor and critic towers of flax's
// ActorCritic with separate torsos (the Gaussian workload's 4 x 256 SiLU
// towers; forward at boonta/networks/network.py:38-49, backward of
// jax.value_and_grad at boonta/algorithms/ppo.py:155-157).
//
// Every row of a minibatch goes through the torso independently, so a
// workgroup that owns 16 rows can run all layers back to back: the forward
// keeps each layer's output in LDS as the next layer's input, and the
// backward keeps each input cotangent in registers for the next LayerNorm
// backward.  Only what the weight gradients and the next launches need goes
// to HBM (Z, Y, mean, rstd forward; dZ and the LayerNorm parameter
// partials backward), and the per-layer launch, prologue and epilogue
// latencies are paid once per torso instead of once per layer.
//
// Tiling (both directions): 16 rows x 256 features per workgroup, four
// waves of 64 features as four 16 x 16 blocks on v_mfma_f32_16x16x4f32;
// block j's column li of wave w is feature 64 w + 4 li + j, so a lane holds
// rows 4 kq + v (v < 4) of four adjacent features and every row access is
// one 16-byte vector.  The forward's contraction and epilogue are those of
// ppo_gemm_ln_act_fwd_f32 (same k order, same statistics), so a chain is
// bit-identical to one fused launch per layer.  The backward's dX = dZ W^T
// reads the layer's kernel transposed (an image the forward writes from the
// parameters it is given, each workgroup a share of its rows), which gives
// its B operand the forward's coalesced row reads.
#include "headloss.h"

using namespace ppo_hl;

namespace {

constexpr int MC_THREADS = 256;
constexpr int MC_ROWS = 16;
constexpr int MC_F = 256;
constexpr int MC_MAXL = 8;
constexpr int SX_PITCH = MC_F + 4;  // LDS row pitch of the 16-row activation tile

__device__ __forceinline__ floatx4 mfma4(const float (&a)[4], const float (&b)[4], floatx4 acc) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
  return acc;
}

struct FwdArgs {
  const float* X;  // layer 0 input rows (row r is X[idx[r]] when idx is non-null)
  int64_t ldx;
  const int32_t* idx;
  int M, K0, L, act;
  float eps;
  int64_t ldw0;  // row pitch of layer 0's kernel [K0][256]; later layers' kernels are [256][ldw]
  int64_t ldw, ld;  // ld: row pitch of Z and Y
  const float* W[MC_MAXL];
  const float* bias[MC_MAXL];
  const float* gamma[MC_MAXL];
  const float* beta[MC_MAXL];
  float* Z[MC_MAXL];
  float* Y[MC_MAXL];
  float* mean[MC_MAXL];
  float* rstd[MC_MAXL];
  float* WT[MC_MAXL];  // layer l >= 1: its kernel transposed [256 out][256 in] (written), or all null
  // tower t's input, parameters, rows (Z, Y), statistics and transposed
  // kernels sit t times these element strides after tower 0's
  int64_t tX, tP, tR, tS, tWT;
};

// One layer's 16 x 256 contraction: acc[j] += A[rows][k] W[k][c4 + j] in the
// k order of the fused per-layer forward (64-deep chunks, each k step of 16
// as four dependent MFMAs).  A comes from global rows (layer 0) or from the
// LDS tile.
// The kernel operands of one 64-deep chunk: w[u][s] = W[k0 + 16 u + 4 kq +
// s][c4 .. c4 + 3].  KC > 0: the kernel's row pitch is MC_F, so the loads
// take one 32-bit lane offset and immediate row offsets from a uniform base
// (with a run-time pitch the compiler keeps sixteen 64-bit lane addresses
// per chunk, which it spills).
template <int KC>
__device__ __forceinline__ void load_w(int k0, floatx4 (&w)[4][4], const float* W, int64_t ldw, int K, int kq,
                                       int c4) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (KC > 0) {
      const float* Wu = W + (k0 + 16 * u) * MC_F;
      const uint32_t lane = (uint32_t)(4 * kq * MC_F + c4);
#pragma unroll
      for (int s = 0; s < 4; ++s) w[u][s] = *reinterpret_cast<const floatx4*>(Wu + lane + s * MC_F);
    } else {
      const int kb = k0 + 16 * u + 4 * kq;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = kb + s;
        w[u][s] = k < K ? *reinterpret_cast<const floatx4*>(W + (int64_t)k * ldw + c4) : floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }
}

// One layer's 16 x 256 contraction: acc[j] += A[rows][k] W[k][c4 + j] in the
// k order of the fused per-layer forward (64-deep chunks, each k step of 16
// as four dependent MFMAs).  A comes from global rows (layer 0) or from the
// LDS tile.  w0: the first chunk's kernel operands, loaded here unless PRE
// (the caller issued them earlier, ahead of its own stores: a wait for a
// load also waits for every store issued before it).
template <int SRC, bool VA, int KC = 0, bool PRE = false>
__device__ __forceinline__ void contract(floatx4 (&acc)[4], const float* xrow, bool a_live, const float* lds_row,
                                         const float* W, int64_t ldw, int K_, int kq, int c4, floatx4 (&w0)[4][4]) {
  // KC > 0: the reduction length is that compile-time constant (the 256-wide
  // layers), so no load is conditional and the prefetches stay in flight
  const int K = KC > 0 ? KC : K_;
  auto load_a = [&](int k0, float (&a)[4][4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int kb = k0 + 16 * u + 4 * kq;
      if (SRC == 1) {
        const floatx4 x4 = kb < K ? *reinterpret_cast<const floatx4*>(lds_row + kb) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) a[u][s] = x4[s];
      } else if (VA) {
        const floatx4 x4 = (a_live && kb < K) ? *reinterpret_cast<const floatx4*>(xrow + kb)
                                                : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) a[u][s] = x4[s];
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) a[u][s] = (a_live && kb + s < K) ? xrow[kb + s] : 0.f;
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
  floatx4 w1[4][4];
  // (on the 256-deep contractions, scheduling barriers keep each chunk's
  // loads issued ahead of the previous chunk's MFMAs; left alone the
  // compiler sinks every load next to its MFMA and only two or three stay
  // in flight)
  auto fence = [] {
    if constexpr (KC > 0) __builtin_amdgcn_sched_barrier(0);
  };
  load_a(0, a0);
  if (!PRE) load_w<KC>(0, w0, W, ldw, K, kq, c4);
  for (int k0 = 0; k0 < K; k0 += 128) {
    if (k0 + 64 < K) {
      load_a(k0 + 64, a1);
      load_w<KC>(k0 + 64, w1, W, ldw, K, kq, c4);
    }
    fence();
    compute(a0, w0);
    fence();
    if (k0 + 64 >= K) break;
    if (k0 + 128 < K) {
      load_a(k0 + 128, a0);
      load_w<KC>(k0 + 128, w0, W, ldw, K, kq, c4);
    }
    fence();
    compute(a1, w1);
    fence();
  }
}

// The fused heads + PPO loss of a pair of separate towers, run by the
// forward chain on its last layer's output: workgroup (x, tower) holds rows
// 16 x .. 16 x + 15 of its tower's last Y in the LDS tile and computes, for
// its tower alone, the head outputs (phase A), the loss terms and the head
// outputs' cotangents (phase B), the head input's cotangent dY — the
// backward chain's input — and the head weight partials (C1, C2).  Every
// operand and operation is that of head_loss_fs_kernel<true, 4, ACT_NONE>
// over the same rows (the head input read from LDS instead of HBM), so the
// results are the same bits; the two towers write disjoint entries of each
// 16-row block's partials.
constexpr int HEAD_NB = MC_F / 64;  // 16-feature blocks per wave in the head phases

// A lane's head parameters for the phases below: the B operands of phase A
// and C1 (actor) or of phase A and the value weights of C1 (critic), read
// from the tower's head kernel [256][ld] that the workgroup copied to LDS
// (hk) at its start.
struct HeadW {
  float wA[HEAD_NB][4], bT[HEAD_NB][4], wcf[HEAD_NB];
};

// Copies the tower's head kernel ([256][ld] floats, 256-byte aligned: ld KB)
// straight into LDS, 1 KB per wave copy; the copies complete in order with
// the chain's own loads.
__device__ __forceinline__ void copy_head_w(const HeadLossParams& hp, bool actor, float* hk) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const char* src = reinterpret_cast<const char*>(actor ? hp.wa : hp.wc);
  const int ld = actor ? (int)hp.ldwa : (int)hp.ldwc;
  for (int c = wave; c < ld; c += MC_THREADS / 64)
    ppo::lds_copy16(src + 1024 * c + 16 * lane, reinterpret_cast<char*>(hk) + 1024 * c);
}

__device__ __forceinline__ void load_head_w(const HeadLossParams& hp, bool actor, const float* hk, HeadW& w) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int kq = lane >> 4;
  const int ja = min(li, (int)hp.ldwa - 1);
#pragma unroll
  for (int i = 0; i < HEAD_NB; ++i) {
    const int fb = 16 * (wave + 4 * i);
    const int f = fb + li;
    w.wcf[i] = actor ? 0.f : hk[f * hp.ldwc];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (actor) {
        w.wA[i][q] = li < hp.na ? hk[(fb + 4 * kq + q) * hp.ldwa + ja] : 0.f;
        w.bT[i][q] = 4 * kq + q < hp.na ? hk[f * hp.ldwa + min(4 * kq + q, (int)hp.ldwa - 1)] : 0.f;
      } else {
        w.wA[i][q] = li == 0 ? hk[(fb + 4 * kq + q) * hp.ldwc] : 0.f;
        w.bT[i][q] = 0.f;
      }
    }
  }
}

template <int PART>
__device__ __forceinline__ void chain_head(const HeadLossParams& hp, const float (*sX)[SX_PITCH],
                                           const LaneIn (&lin)[1], const HeadW& w, float (*s_part)[MC_ROWS][LDO],
                                           float (*s_dout)[LDO], double (*s_st)[NSTAT], float (*s_dsc)[16]) {
  constexpr bool ACTOR = PART == PART_ACTOR;
  constexpr int NB = HEAD_NB;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int kq = lane >> 4;
  const int r0 = blockIdx.x * MC_ROWS;
  const int64_t blk = blockIdx.x;
  const int last = hp.rows - 1;
  const ColConst cc = load_cols(hp, true, threadIdx.x & 15);
  const bool liveA = r0 + li < hp.rows;
  int64_t rowq[4];
  bool liveq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    liveq[q] = r0 + 4 * kq + q < hp.rows;
    rowq[q] = min(r0 + 4 * kq + q, last);
  }
  const floatx4 z4 = {0.f, 0.f, 0.f, 0.f};
  floatx4 hA[NB];
  float h2[NB][4];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int fb = 16 * (wave + 4 * i);
    const int f = fb + li;
    hA[i] = liveA ? *reinterpret_cast<const floatx4*>(&sX[li][fb + 4 * kq]) : z4;
#pragma unroll
    for (int q = 0; q < 4; ++q) h2[i][q] = liveq[q] ? sX[4 * kq + q][f] : 0.f;
  }

  // A. per-wave partial head outputs of the 16 rows
  {
    floatx4 acc = z4;
#pragma unroll
    for (int i = 0; i < NB; ++i) acc = ppo_hl::mfma4(hA[i], w.wA[i], acc);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (ACTOR) s_part[wave][4 * kq + v][li] = acc[v];
      else if (li == 0) s_part[wave][4 * kq + v][16] = acc[v];
    }
  }
  __syncthreads();

  // B. this tower's loss terms and head-output cotangents
  phase_b<MC_ROWS, 4, true, 16, PART>(hp, blk, s_part, s_dout, s_st, s_dsc, lin, cc);

  // C1. the head input's cotangent; C2. the head weight gradient partial
  if (ACTOR) {
    const floatx4 dv4 = *reinterpret_cast<const floatx4*>(&s_dout[li][4 * kq]);
    const floatx4 a_in = liveA ? dv4 : z4;
    float dq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) dq[q] = s_dout[4 * kq + q][li];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int fb = 16 * (wave + 4 * i);
      const int f = fb + li;
      const floatx4 g = ppo_hl::mfma4(a_in, w.bT[i], z4);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (liveq[v]) hp.dha[rowq[v] * hp.lddha + f] = g[v];
      const floatx4 gw = ppo_hl::mfma4(floatx4{h2[i][0], h2[i][1], h2[i][2], h2[i][3]}, dq, z4);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (li < (int)hp.ldwa) hp.wpart_a[(blk * MC_F + fb + 4 * kq + v) * hp.ldwa + li] = gw[v];
    }
  } else {
    float dvq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) dvq[q] = s_dout[4 * kq + q][16];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int fb = 16 * (wave + 4 * i);
      const int f = fb + li;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (liveq[v]) hp.dhc[rowq[v] * hp.lddhc + f] = dvq[v] * w.wcf[i];
      float wv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) wv[q] = li == 0 ? dvq[q] : 0.f;
      const floatx4 gc = ppo_hl::mfma4(floatx4{h2[i][0], h2[i][1], h2[i][2], h2[i][3]}, wv, z4);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (li < (int)hp.ldwc) hp.wpart_c[(blk * MC_F + fb + 4 * kq + v) * hp.ldwc + li] = li == 0 ? gc[v] : 0.f;
    }
  }
}

// ACT: the activation as a compile-time constant, so that the epilogue holds
// only its code (a run-time switch per element interleaves every case's code,
// tanhf's included, through the loop and the taken path thrashes the
// instruction cache)
// HEAD: the fused heads + loss of a pair of towers on the last layer's output
// (chain_head; hp is unused otherwise).
template <bool VA, int ACT, bool HEAD>
__device__ __forceinline__ void mlp_ln_fwd_body(const FwdArgs& p, const HeadLossParams& hp) {
  __shared__ __attribute__((aligned(16))) float sX[MC_ROWS][SX_PITCH];
  __shared__ __attribute__((aligned(16))) float s_part[HEAD ? 4 : 1][MC_ROWS][LDO];
  __shared__ __attribute__((aligned(16))) float s_dout[HEAD ? MC_ROWS : 1][LDO];
  __shared__ double s_st[HEAD ? MC_ROWS : 1][NSTAT];
  __shared__ float s_dsc[HEAD ? MC_ROWS : 1][16];
  __shared__ __attribute__((aligned(1024))) float s_hk[HEAD ? MC_F * 16 : 1];  // the tower's head kernel
  __shared__ float s_sum[4][MC_ROWS];
  __shared__ float s_sq[4][MC_ROWS];
  const int64_t t = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int kq = lane >> 4;
  const int r0 = blockIdx.x * MC_ROWS;
  const int ra = r0 + li;
  const bool a_live = ra < p.M;
  const float* X = p.X + t * p.tX;
  const float* xrow = X + (a_live ? (int64_t)(p.idx ? p.idx[ra] : ra) * p.ldx : 0);
  const int c4 = 64 * wave + 4 * li;
  // the head loss's sample indices (thread: row threadIdx.x / 16, column
  // threadIdx.x % 16); their gathers are issued with the last layer
  LaneIn lin[1];
  if constexpr (HEAD) {
    lane_samples(hp, r0, threadIdx.x, lin);
    copy_head_w(hp, t == 0, s_hk);
  }

  // layer l's bias, scale and offset for this lane's features, and (l >= 1)
  // the first chunk of its kernel: issued during layer l - 1, ahead of its
  // stores
  auto params = [&](int l, floatx4& bias4, floatx4& g4, floatx4& be4) {
    const float* bias = p.bias[l] ? p.bias[l] + t * p.tP : nullptr;
    bias4 = bias ? *reinterpret_cast<const floatx4*>(bias + c4) : floatx4{0.f, 0.f, 0.f, 0.f};
    g4 = *reinterpret_cast<const floatx4*>(p.gamma[l] + t * p.tP + c4);
    be4 = *reinterpret_cast<const floatx4*>(p.beta[l] + t * p.tP + c4);
  };
  floatx4 bias4, g4, be4;
  params(0, bias4, g4, be4);
  floatx4 w0[4][4];

  // this workgroup's share of the transposed kernels of layers 1.. (the
  // backward's dX reads them): 32 x 32 tiles of WT_l[o][k] = W_l[k][o],
  // tiles blockIdx.x + i gridDim.x of the (L - 1) x 64 of a tower.  Up to
  // WT_EARLY tiles per workgroup: each thread loads one 16-byte run of a
  // tile row here, puts it in an LDS tile after the first layer's
  // contraction and writes a 16-byte run of the transposed tile after that
  // layer's statistics barrier (loads and stores coalesced, off the chain's
  // path); more tiles go through a loop at the end of the kernel.
  constexpr int WT_EARLY = 2;
  __shared__ float s_tile[WT_EARLY][32][33];
  const int nwg = gridDim.x;
  const int wt_tiles = p.WT[1] != nullptr ? (p.L - 1) * 64 : 0;
  const int wt_mine = wt_tiles > (int)blockIdx.x ? (wt_tiles - 1 - (int)blockIdx.x) / nwg + 1 : 0;
  const bool wt_early = wt_mine <= WT_EARLY;
  const int tr_row = threadIdx.x >> 3, tr_q = threadIdx.x & 7;   // tile row / 16-byte run of it
  // W_l or WT_l of layer ll (read through compile-time indices: a run-time
  // index into the argument arrays would put them in scratch)
  auto wl = [&](int ll) {
    const float* r = nullptr;
#pragma unroll
    for (int q = 1; q < MC_MAXL; ++q)
      if (q == ll) r = p.W[q];
    return r + t * p.tP;
  };
  auto wtl = [&](int ll) {
    float* r = nullptr;
#pragma unroll
    for (int q = 1; q < MC_MAXL; ++q)
      if (q == ll) r = p.WT[q];
    return r + t * p.tWT;
  };
  // tile id -> layer, 32-row block of k, 32-column block of o
  auto tile_src = [&](int id) {
    const int ll = 1 + id / 64, tk = (id & 63) >> 3, to = id & 7;
    return wl(ll) + (int64_t)(32 * tk + tr_row) * MC_F + 32 * to + 4 * tr_q;
  };
  auto tile_dst = [&](int id) {
    const int ll = 1 + id / 64, tk = (id & 63) >> 3, to = id & 7;
    return wtl(ll) + (int64_t)(32 * to + tr_row) * MC_F + 32 * tk + 4 * tr_q;
  };
  floatx4 tv[WT_EARLY];
  if (wt_early) {
#pragma unroll
    for (int i = 0; i < WT_EARLY; ++i)
      if (i < wt_mine) tv[i] = *reinterpret_cast<const floatx4*>(tile_src(blockIdx.x + i * nwg));
  }
  // the transposed run of tile i this thread writes: o = row, k = 4 q .. 4 q + 3
  auto tile_out = [&](int i) {
    return floatx4{s_tile[i][4 * tr_q][tr_row], s_tile[i][4 * tr_q + 1][tr_row], s_tile[i][4 * tr_q + 2][tr_row],
                   s_tile[i][4 * tr_q + 3][tr_row]};
  };

  for (int l = 0; l < p.L; ++l) {
    const float* W = p.W[l] + t * p.tP;
    if constexpr (HEAD) {
      if (l == p.L - 1) lane_gathers(hp, threadIdx.x & 15, lin);
    }
    floatx4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (l == 0)
      contract<0, VA>(acc, xrow, a_live, nullptr, W, p.ldw0, p.K0, kq, c4, w0);
    else
      contract<1, true, MC_F, true>(acc, nullptr, true, &sX[li][0], W, MC_F, MC_F, kq, c4, w0);

    float z[4][4];
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
    if (l == 0 && wt_early) {
#pragma unroll
      for (int i = 0; i < WT_EARLY; ++i)
        if (i < wt_mine)
#pragma unroll
          for (int e = 0; e < 4; ++e) s_tile[i][tr_row][4 * tr_q + e] = tv[i][e];
    }
    const floatx4 gl = g4, bel = be4;
    if (l + 1 < p.L) {
      load_w<MC_F>(0, w0, p.W[l + 1] + t * p.tP, MC_F, MC_F, kq, c4);
      params(l + 1, bias4, g4, be4);
    }
    // every wave is past its contraction (its reads of sX) once here
    __syncthreads();
    if (l == 0 && wt_early) {
#pragma unroll
      for (int i = 0; i < WT_EARLY; ++i)
        if (i < wt_mine) *reinterpret_cast<floatx4*>(tile_dst(blockIdx.x + i * nwg)) = tile_out(i);
    }
    float* Zl = p.Z[l] + t * p.tR;
    float* Yl = p.Y[l] + t * p.tR;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int rr = 4 * kq + v;
      const int row = r0 + rr;
      const float s = (s_sum[0][rr] + s_sum[1][rr]) + (s_sum[2][rr] + s_sum[3][rr]);
      const float s2 = (s_sq[0][rr] + s_sq[1][rr]) + (s_sq[2][rr] + s_sq[3][rr]);
      float mean, rstd;
      ppo::ln_stats256(s, s2, p.eps, mean, rstd);
      floatx4 zo, yo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        zo[j] = z[v][j];
        yo[j] = ppo::act_fwd(ACT, ppo::ln_apply(z[v][j], mean, rstd, gl[j], bel[j]));
      }
      if (HEAD || l + 1 < p.L) *reinterpret_cast<floatx4*>(&sX[rr][c4]) = yo;
      if (row >= p.M) continue;
      if (wave == 0 && li == 0) {
        p.mean[l][t * p.tS + row] = mean;
        p.rstd[l][t * p.tS + row] = rstd;
      }
      *reinterpret_cast<floatx4*>(Zl + (int64_t)row * p.ld + c4) = zo;
      *reinterpret_cast<floatx4*>(Yl + (int64_t)row * p.ld + c4) = yo;
    }
    // the next layer's contraction reads the tile (and s_sum is rewritten)
    __syncthreads();
  }
  if constexpr (HEAD) {
    // the head kernel's copies, issued first, are long complete: wait for
    // them explicitly (the compiler does not track them), then meet
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    HeadW hw;
    load_head_w(hp, t == 0, s_hk, hw);
    if (t == 0) chain_head<PART_ACTOR>(hp, sX, lin, hw, s_part, s_dout, s_st, s_dsc);
    else chain_head<PART_CRITIC>(hp, sX, lin, hw, s_part, s_dout, s_st, s_dsc);
  }
  if (!wt_early) {
    for (int i = 0; i < wt_mine; ++i) {
      const int id = blockIdx.x + i * nwg;
      const floatx4 v = *reinterpret_cast<const floatx4*>(tile_src(id));
#pragma unroll
      for (int e = 0; e < 4; ++e) s_tile[0][tr_row][4 * tr_q + e] = v[e];
      __syncthreads();
      *reinterpret_cast<floatx4*>(tile_dst(id)) = tile_out(0);
      __syncthreads();
    }
  }
}

template <bool VA, int ACT, bool HEAD>
__global__ void __launch_bounds__(MC_THREADS) mlp_ln_fwd_kernel(FwdArgs p, HeadLossParams hp) {
  mlp_ln_fwd_body<VA, ACT, HEAD>(p, hp);
}

struct BwdArgs {
  const float* dY;  // cotangent of the last layer's output
  int64_t lddy;
  int M, L, act;
  int64_t ld;       // row pitch of Z and dZ
  int64_t ldwt;     // row pitch of the transposed kernels
  const float* Z[MC_MAXL];
  const float* mean[MC_MAXL];
  const float* rstd[MC_MAXL];
  const float* gamma[MC_MAXL];
  const float* beta[MC_MAXL];
  const float* WT[MC_MAXL];  // layer l >= 1: its kernel transposed, WT[out][in]
  float* dZ[MC_MAXL];
  float* part[MC_MAXL];      // [blocks][2 F]: scale | bias gradient sums of the block's rows
  int64_t tR, tS, tP, tWT, tPart;
};

template <int ACT>
__device__ __forceinline__ void mlp_ln_bwd_body(const BwdArgs& p) {
  __shared__ float sX[MC_ROWS][SX_PITCH];
  __shared__ float s_sum[4][MC_ROWS];
  __shared__ float s_sq[4][MC_ROWS];
  const int64_t t = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int kq = lane >> 4;
  const int r0 = blockIdx.x * MC_ROWS;
  const int c4 = 64 * wave + 4 * li;

  // the cotangent of the current layer's output: rows 4 kq + v, features c4 + j
  float dy[4][4];
  {
    const float* dY = p.dY + t * p.tR;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = r0 + 4 * kq + v;
      const floatx4 d = row < p.M ? *reinterpret_cast<const floatx4*>(dY + (int64_t)row * p.lddy + c4)
                                  : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) dy[v][j] = d[j];
    }
  }

  // layer l's LayerNorm operands for this lane (Z at rows 4 kq + v, their
  // statistics, scale and offset): issued during layer l + 1 before its dX
  // contraction, and the first chunk of that contraction's kernel ahead of
  // layer l + 1's stores
  floatx4 zz[4], g4, be4;
  float mu[4], rs[4];
  auto ln_ops = [&](int l) {
    const float* Zl = p.Z[l] + t * p.tR;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = r0 + 4 * kq + v;
      const int rr = row < p.M ? row : r0;
      zz[v] = *reinterpret_cast<const floatx4*>(Zl + (int64_t)rr * p.ld + c4);
      mu[v] = p.mean[l][t * p.tS + rr];
      rs[v] = p.rstd[l][t * p.tS + rr];
    }
    g4 = *reinterpret_cast<const floatx4*>(p.gamma[l] + t * p.tP + c4);
    be4 = *reinterpret_cast<const floatx4*>(p.beta[l] + t * p.tP + c4);
  };
  ln_ops(p.L - 1);
  floatx4 w0[4][4];

  for (int l = p.L - 1; l >= 0; --l) {
    float xh[4][4], g[4][4], rsl[4];
    float sg[4], sgx[4];
    float pg[4] = {0.f, 0.f, 0.f, 0.f}, pb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = r0 + 4 * kq + v;
      const bool live = row < p.M;
      rsl[v] = rs[v];
      sg[v] = 0.f;
      sgx[v] = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xh[v][j] = live ? (zz[v][j] - mu[v]) * rs[v] : 0.f;
        // the forward's normalised value, rounded as the forward rounded it
        const float yl = ppo::ln_apply(zz[v][j], mu[v], rs[v], g4[j], be4[j]);
        const float a = (ACT == ACT_RELU || ACT == ACT_TANH) ? ppo::act_fwd(ACT, yl) : yl;
        const float dyl = live ? dy[v][j] * ppo::act_grad(ACT, a) : 0.f;
        pg[j] += dyl * xh[v][j];
        pb[j] += dyl;
        g[v][j] = dyl * g4[j];
        sg[v] += g[v][j];
        sgx[v] += g[v][j] * xh[v][j];
      }
      sg[v] = ppo::sum16(sg[v]);
      sgx[v] = ppo::sum16(sgx[v]);
    }
    if (li == 0) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        s_sum[wave][4 * kq + v] = sg[v];
        s_sq[wave][4 * kq + v] = sgx[v];
      }
    }
    // LayerNorm parameter partials: this block's rows, summed in a fixed
    // order (the lane's four rows, then the four row groups)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pg[j] = ppo::add_xor16(pg[j]);
      pb[j] = ppo::add_xor16(pb[j]);
      pg[j] = ppo::add_xor32(pg[j]);
      pb[j] = ppo::add_xor32(pb[j]);
    }
    if (l > 0) load_w<MC_F>(0, w0, p.WT[l] + t * p.tWT, MC_F, MC_F, kq, c4);
    if (kq == 0) {
      float* part = p.part[l] + t * p.tPart + (int64_t)blockIdx.x * 2 * MC_F;
      *reinterpret_cast<floatx4*>(part + c4) = floatx4{pg[0], pg[1], pg[2], pg[3]};
      *reinterpret_cast<floatx4*>(part + MC_F + c4) = floatx4{pb[0], pb[1], pb[2], pb[3]};
    }
    // every wave is past the previous dX contraction (its reads of sX) here
    __syncthreads();
    float* dZl = p.dZ[l] + t * p.tR;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int rr = 4 * kq + v;
      const int row = r0 + rr;
      const float s = ((s_sum[0][rr] + s_sum[1][rr]) + (s_sum[2][rr] + s_sum[3][rr])) / (float)MC_F;
      const float s2 = ((s_sq[0][rr] + s_sq[1][rr]) + (s_sq[2][rr] + s_sq[3][rr])) / (float)MC_F;
      floatx4 d;
#pragma unroll
      for (int j = 0; j < 4; ++j) d[j] = row < p.M ? rsl[v] * (g[v][j] - s - xh[v][j] * s2) : 0.f;
      if (l > 0) *reinterpret_cast<floatx4*>(&sX[rr][c4]) = d;
      if (row < p.M) *reinterpret_cast<floatx4*>(dZl + (int64_t)row * p.ld + c4) = d;
    }
    if (l == 0) break;
    __syncthreads();
    ln_ops(l - 1);
    // dY of layer l - 1 = dZ_l W_l^T, from the transposed kernel WT_l[out][in]
    floatx4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    contract<1, true, MC_F, true>(acc, nullptr, true, &sX[li][0], p.WT[l] + t * p.tWT, MC_F, MC_F, kq, c4, w0);
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int j = 0; j < 4; ++j) dy[v][j] = acc[j][v];
  }
}

template <int ACT>
__global__ void __launch_bounds__(MC_THREADS) mlp_ln_bwd_kernel(BwdArgs p) {
  mlp_ln_bwd_body<ACT>(p);
}

// The forward chain with the fused heads + loss, then the backward chain, in
// one launch: every row's loss cotangent depends only on that row, so the
// workgroup that owns 16 rows of a tower runs their backward right after
// their forward.  The backward's input cotangents, Z and statistics are this
// workgroup's own stores (complete and visible to its waves after the wait
// and barrier below); the transposed kernels it reads were written before
// the launch (the forward part writes none).
template <bool VA, int ACT>
__global__ void __launch_bounds__(MC_THREADS) mlp_ln_fwd_bwd_kernel(FwdArgs p, HeadLossParams hp, BwdArgs b) {
  mlp_ln_fwd_body<VA, ACT, true>(p, hp);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  mlp_ln_bwd_body<ACT>(b);
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

PPO_EXPORT int ppo_mlp_chain_max_layers() { return MC_MAXL; }

// Forward of L Dense(256) -> LayerNorm -> activation layers for `towers`
// towers in one launch (see the top of this file); arrays hold tower 0's
// per-layer pointers.
// Checks the chain forward's arguments (messages under `name`) and fills a.
static int chain_fwd_setup(FwdArgs& a, bool& va, const char* name, int towers, int L, const float* X, int64_t ldx,
                           const int32_t* rows_idx, int M, int K0, const float* const* W, int64_t ldw0, int64_t ldw,
                           const float* const* bias, const float* const* gamma, const float* const* beta,
                           float* const* Z, float* const* Y, int64_t ld, float* const* mean, float* const* rstd,
                           float eps, int act, int64_t stride_x, int64_t stride_params, int64_t stride_rows,
                           int64_t stride_stats, float* const* WT, int64_t stride_wt) {
  if (towers < 1 || towers > 8 || L < 1 || L > MC_MAXL || M < 0 || K0 < 1 || act < 0 || act > 3 || ldx < K0 ||
      ldw0 < MC_F || ldw != MC_F || ld < MC_F || !W || !bias || !gamma || !beta || !Z || !Y || !mean || !rstd ||
      ldw0 % 4 || ldw % 4 || ld % 4 || (towers > 1 && (stride_x % 4 || stride_params % 4 || stride_rows % 4)))
    return ppo::set_error(PPO_ERR_ARG, "%s: bad argument (towers=%d L=%d M=%d K0=%d)", name, towers, L, M, K0);
  a = FwdArgs{};
  a.X = X; a.ldx = ldx; a.idx = rows_idx; a.M = M; a.K0 = K0; a.L = L; a.act = act; a.eps = eps;
  a.ldw0 = ldw0; a.ldw = ldw; a.ld = ld;
  a.tX = stride_x; a.tP = stride_params; a.tR = stride_rows; a.tS = stride_stats; a.tWT = stride_wt;
  if (!X) return ppo::set_error(PPO_ERR_ARG, "%s: null input", name);
  if (WT && L > 1) {
    if (towers > 1 && stride_wt % 4) return ppo::set_error(PPO_ERR_ARG, "%s: bad WT stride", name);
    for (int l = 1; l < L; ++l) {
      if (!WT[l] || !aligned16(WT[l]))
        return ppo::set_error(PPO_ERR_ARG, "%s: layer %d needs a 16-byte aligned WT", name, l);
      a.WT[l] = WT[l];
    }
  }
  for (int l = 0; l < L; ++l) {
    if (!W[l] || !gamma[l] || !beta[l] || !Z[l] || !Y[l] || !mean[l] || !rstd[l] || !aligned16(W[l]) ||
        (bias[l] && !aligned16(bias[l])) || !aligned16(gamma[l]) || !aligned16(beta[l]) || !aligned16(Z[l]) ||
        !aligned16(Y[l]))
      return ppo::set_error(PPO_ERR_ARG, "%s: layer %d needs 16-byte aligned buffers", name, l);
    a.W[l] = W[l]; a.bias[l] = bias[l]; a.gamma[l] = gamma[l]; a.beta[l] = beta[l];
    a.Z[l] = Z[l]; a.Y[l] = Y[l]; a.mean[l] = mean[l]; a.rstd[l] = rstd[l];
  }
  va = aligned16(X) && ldx % 4 == 0 && K0 % 4 == 0 && (towers == 1 || stride_x % 4 == 0);
  return PPO_OK;
}

template <bool HEAD>
static void chain_fwd_launch(hipStream_t st, const FwdArgs& a, const HeadLossParams& hp, bool va, int towers) {
  const dim3 grid(ppo::ceil_div(a.M, MC_ROWS), towers), block(MC_THREADS);
#define PPO_CHAIN_FWD(ACTV)                                                                          \
  if (va) hipLaunchKernelGGL((mlp_ln_fwd_kernel<true, ACTV, HEAD>), grid, block, 0, st, a, hp);     \
  else hipLaunchKernelGGL((mlp_ln_fwd_kernel<false, ACTV, HEAD>), grid, block, 0, st, a, hp);
  switch (a.act) {
    case ACT_RELU: PPO_CHAIN_FWD(ACT_RELU) break;
    case ACT_TANH: PPO_CHAIN_FWD(ACT_TANH) break;
    case ACT_SILU: PPO_CHAIN_FWD(ACT_SILU) break;
    default: PPO_CHAIN_FWD(ACT_NONE) break;
  }
#undef PPO_CHAIN_FWD
}

PPO_EXPORT int ppo_mlp_ln_fwd_f32(void* stream, int towers, int L, const float* X, int64_t ldx,
                                 const int32_t* rows_idx, int M, int K0, const float* const* W, int64_t ldw0,
                                 int64_t ldw, const float* const* bias, const float* const* gamma,
                                 const float* const* beta, float* const* Z, float* const* Y, int64_t ld,
                                 float* const* mean, float* const* rstd, float eps, int act, int64_t stride_x,
                                 int64_t stride_params, int64_t stride_rows, int64_t stride_stats,
                                 float* const* WT, int64_t stride_wt) {
  FwdArgs a;
  bool va = false;
  const int rc = chain_fwd_setup(a, va, "ppo_mlp_ln_fwd_f32", towers, L, X, ldx, rows_idx, M, K0, W, ldw0, ldw, bias,
                                 gamma, beta, Z, Y, ld, mean, rstd, eps, act, stride_x, stride_params, stride_rows,
                                 stride_stats, WT, stride_wt);
  if (rc != PPO_OK) return rc;
  if (M == 0) return PPO_OK;
  chain_fwd_launch<false>(ppo::as_stream(stream), a, HeadLossParams{}, va, towers);
  return ppo::check_launch("ppo_mlp_ln_fwd_f32");
}

extern "C" int ppo_head_loss_blocks(int rows);

// The forward chain of an actor / critic pair (towers = 2) followed by their
// fused heads + PPO loss in the same launch: the results of
// ppo_mlp_ln_fwd_f32(<chain arguments>) then ppo_head_loss_f32(<head
// arguments>), bit for bit, where the head inputs are the chain's last
// outputs (ha = Y[L - 1], hc = ha + stride_rows, ldha = ldhc = ld), the
// heads are separate (hc non-null) over F = 256 features with no activation
// derivative (act_a = act_c = 0), rows = M, and M is small enough that the
// head loss's partials are kept per 16-row block.
PPO_EXPORT int ppo_mlp_ln_fwd_head_loss_f32(
    void* stream, int towers, int L, const float* X, int64_t ldx, const int32_t* rows_idx, int M, int K0,
    const float* const* W, int64_t ldw0, int64_t ldw, const float* const* bias, const float* const* gamma,
    const float* const* beta, float* const* Z, float* const* Y, int64_t ld, float* const* mean, float* const* rstd,
    float eps, int act, int64_t stride_x, int64_t stride_params, int64_t stride_rows, int64_t stride_stats,
    float* const* WT, int64_t stride_wt, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha,
    const float* wa, int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc,
    int64_t ldwc, const float* bc, int F, int A, const float* scale_param, const int32_t* action_i,
    const float* action_f, const float* old_logp, const float* old_value, const float* adv, const float* ret,
    int act_a, const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature, int64_t sample_stride) {
  const char* name = "ppo_mlp_ln_fwd_head_loss_f32";
  FwdArgs a;
  bool va = false;
  int rc = chain_fwd_setup(a, va, name, towers, L, X, ldx, rows_idx, M, K0, W, ldw0, ldw, bias, gamma, beta, Z, Y,
                           ld, mean, rstd, eps, act, stride_x, stride_params, stride_rows, stride_stats, WT,
                           stride_wt);
  if (rc != PPO_OK) return rc;
  HeadLossParams hp;
  rc = head_loss_setup(hp, name, dist, rows, idx, ha, ldha, wa, ldwa, ba, na, hc, ldhc, wc, ldwc, bc, F, A,
                       scale_param, action_i, action_f, old_logp, old_value, adv, ret, act_a, aux_a, ldaux_a, dha,
                       lddha, act_c, aux_c, ldaux_c, dhc, lddhc, wpart_a, bpart_a, wpart_c, bpart_c, dscale_partial,
                       stats_partial, clip_eps, clip_value_loss, ent_coef, vf_coef, temperature, nullptr, 1, 1,
                       sample_stride);
  if (rc != PPO_OK) return rc;
  if (towers != 2 || !hc || F != MC_F || act_a != ACT_NONE || act_c != ACT_NONE || rows != M || ha != Y[L - 1] ||
      hc != Y[L - 1] + stride_rows || ldha != ld || ldhc != ld || (reinterpret_cast<uintptr_t>(wa) & 255) ||
      (reinterpret_cast<uintptr_t>(wc) & 255) ||
      (M > 0 && ppo_head_loss_blocks(M) != ppo::ceil_div(M, MC_ROWS)))
    return ppo::set_error(PPO_ERR_ARG, "%s: the heads must read the last layer of both towers (towers=%d F=%d "
                          "rows=%d M=%d)", name, towers, F, rows, M);
  if (M == 0) return PPO_OK;
  chain_fwd_launch<true>(ppo::as_stream(stream), a, hp, va, towers);
  return ppo::check_launch(name);
}

PPO_EXPORT int ppo_mlp_ln_bwd_blocks(int rows) { return rows > 0 ? ppo::ceil_div(rows, MC_ROWS) : 0; }

// Backward of the same chain: from the last layer's output cotangent dY,
// each layer's LayerNorm + activation backward (dZ, and the scale | bias
// gradient partials of each 16-row block) and, below the top, the input
// cotangent dZ W^T through the transposed kernels WT[l] (l >= 1).
PPO_EXPORT int ppo_mlp_ln_bwd_f32(void* stream, int towers, int L, const float* dY, int64_t lddy, int M,
                                 const float* const* Z, const float* const* mean, const float* const* rstd,
                                 const float* const* gamma, const float* const* beta, const float* const* WT,
                                 int64_t ldwt, float* const* dZ, int64_t ld, float* const* partial, int act,
                                 int64_t stride_rows, int64_t stride_stats, int64_t stride_params,
                                 int64_t stride_wt, int64_t stride_part) {
  if (towers < 1 || towers > 8 || L < 1 || L > MC_MAXL || M < 0 || act < 0 || act > 3 || lddy < MC_F ||
      ld < MC_F || ldwt != MC_F || !dY || !Z || !mean || !rstd || !gamma || !beta || !WT || !dZ || !partial ||
      lddy % 4 || ld % 4 || ldwt % 4 ||
      (towers > 1 && (stride_rows % 4 || stride_params % 4 || stride_wt % 4 || stride_part % 4)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_mlp_ln_bwd_f32: bad argument (towers=%d L=%d M=%d)", towers, L, M);
  if (M == 0) return PPO_OK;
  BwdArgs a{};
  a.dY = dY; a.lddy = lddy; a.M = M; a.L = L; a.act = act; a.ld = ld; a.ldwt = ldwt;
  a.tR = stride_rows; a.tS = stride_stats; a.tP = stride_params; a.tWT = stride_wt; a.tPart = stride_part;
  if (!aligned16(dY)) return ppo::set_error(PPO_ERR_ARG, "ppo_mlp_ln_bwd_f32: dY needs 16-byte rows");
  for (int l = 0; l < L; ++l) {
    if (!Z[l] || !mean[l] || !rstd[l] || !gamma[l] || !beta[l] || !dZ[l] || !partial[l] || (l > 0 && !WT[l]) ||
        !aligned16(Z[l]) || !aligned16(gamma[l]) || !aligned16(beta[l]) || !aligned16(dZ[l]) ||
        !aligned16(partial[l]) || (l > 0 && !aligned16(WT[l])))
      return ppo::set_error(PPO_ERR_ARG, "ppo_mlp_ln_bwd_f32: layer %d needs 16-byte aligned buffers", l);
    a.Z[l] = Z[l]; a.mean[l] = mean[l]; a.rstd[l] = rstd[l]; a.gamma[l] = gamma[l]; a.beta[l] = beta[l];
    a.WT[l] = l > 0 ? WT[l] : nullptr; a.dZ[l] = dZ[l]; a.part[l] = partial[l];
  }
  const dim3 grid(ppo::ceil_div(M, MC_ROWS), towers), block(MC_THREADS);
  switch (act) {
    case ACT_RELU: hipLaunchKernelGGL(mlp_ln_bwd_kernel<ACT_RELU>, grid, block, 0, ppo::as_stream(stream), a); break;
    case ACT_TANH: hipLaunchKernelGGL(mlp_ln_bwd_kernel<ACT_TANH>, grid, block, 0, ppo::as_stream(stream), a); break;
    case ACT_SILU: hipLaunchKernelGGL(mlp_ln_bwd_kernel<ACT_SILU>, grid, block, 0, ppo::as_stream(stream), a); break;
    default: hipLaunchKernelGGL(mlp_ln_bwd_kernel<ACT_NONE>, grid, block, 0, ppo::as_stream(stream), a); break;
  }
  return ppo::check_launch("ppo_mlp_ln_bwd_f32");
}

// ppo_mlp_ln_fwd_head_loss_f32 followed by ppo_mlp_ln_bwd_f32 from the heads'
// input cotangents, in one launch, bit for bit: the chain and head arguments
// are those of ppo_mlp_ln_fwd_head_loss_f32, except that WT / stride_wt are
// the transposed kernels the backward reads (layers 1..L-1, [256][256], made
// before this launch, e.g. by ppo_adam_clip_wt_f32; none are written here);
// the backward's dY is dha (tower 1: dhc = dha + stride_rows, lddhc = lddha),
// and it writes dZ (pitch ld) and the LayerNorm parameter partials
// (partial[l], tower stride stride_part) as ppo_mlp_ln_bwd_f32 does.
PPO_EXPORT int ppo_mlp_ln_fwd_head_loss_bwd_f32(
    void* stream, int towers, int L, const float* X, int64_t ldx, const int32_t* rows_idx, int M, int K0,
    const float* const* W, int64_t ldw0, int64_t ldw, const float* const* bias, const float* const* gamma,
    const float* const* beta, float* const* Z, float* const* Y, int64_t ld, float* const* mean, float* const* rstd,
    float eps, int act, int64_t stride_x, int64_t stride_params, int64_t stride_rows, int64_t stride_stats,
    float* const* WT, int64_t stride_wt, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha,
    const float* wa, int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc,
    int64_t ldwc, const float* bc, int F, int A, const float* scale_param, const int32_t* action_i,
    const float* action_f, const float* old_logp, const float* old_value, const float* adv, const float* ret,
    int act_a, const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature, int64_t sample_stride, float* const* dZ, float* const* partial,
    int64_t stride_part) {
  const char* name = "ppo_mlp_ln_fwd_head_loss_bwd_f32";
  FwdArgs a;
  bool va = false;
  // the forward part writes no transposed kernels
  int rc = chain_fwd_setup(a, va, name, towers, L, X, ldx, rows_idx, M, K0, W, ldw0, ldw, bias, gamma, beta, Z, Y,
                           ld, mean, rstd, eps, act, stride_x, stride_params, stride_rows, stride_stats, nullptr, 0);
  if (rc != PPO_OK) return rc;
  HeadLossParams hp;
  rc = head_loss_setup(hp, name, dist, rows, idx, ha, ldha, wa, ldwa, ba, na, hc, ldhc, wc, ldwc, bc, F, A,
                       scale_param, action_i, action_f, old_logp, old_value, adv, ret, act_a, aux_a, ldaux_a, dha,
                       lddha, act_c, aux_c, ldaux_c, dhc, lddhc, wpart_a, bpart_a, wpart_c, bpart_c, dscale_partial,
                       stats_partial, clip_eps, clip_value_loss, ent_coef, vf_coef, temperature, nullptr, 1, 1,
                       sample_stride);
  if (rc != PPO_OK) return rc;
  if (towers != 2 || !hc || F != MC_F || act_a != ACT_NONE || act_c != ACT_NONE || rows != M || ha != Y[L - 1] ||
      hc != Y[L - 1] + stride_rows || ldha != ld || ldhc != ld || (reinterpret_cast<uintptr_t>(wa) & 255) ||
      (reinterpret_cast<uintptr_t>(wc) & 255) ||
      (M > 0 && ppo_head_loss_blocks(M) != ppo::ceil_div(M, MC_ROWS)))
    return ppo::set_error(PPO_ERR_ARG, "%s: the heads must read the last layer of both towers (towers=%d F=%d "
                          "rows=%d M=%d)", name, towers, F, rows, M);
  if (!dha || dhc != dha + stride_rows || lddhc != lddha || lddha < MC_F || lddha % 4 || !aligned16(dha) || !dZ ||
      !partial || stride_part % 4 || (L > 1 && (!WT || stride_wt % 4)))
    return ppo::set_error(PPO_ERR_ARG, "%s: the backward reads dha and dhc = dha + stride_rows; it needs dZ, "
                          "partial and (L > 1) WT tables", name);
  BwdArgs b{};
  b.dY = dha; b.lddy = lddha; b.M = M; b.L = L; b.act = act; b.ld = ld; b.ldwt = MC_F;
  b.tR = stride_rows; b.tS = stride_stats; b.tP = stride_params; b.tWT = stride_wt; b.tPart = stride_part;
  for (int l = 0; l < L; ++l) {
    if (!dZ[l] || !partial[l] || (l > 0 && (!WT[l] || !aligned16(WT[l]))) || !aligned16(dZ[l]) ||
        !aligned16(partial[l]))
      return ppo::set_error(PPO_ERR_ARG, "%s: layer %d needs 16-byte aligned backward buffers", name, l);
    b.Z[l] = Z[l]; b.mean[l] = mean[l]; b.rstd[l] = rstd[l]; b.gamma[l] = gamma[l]; b.beta[l] = beta[l];
    b.WT[l] = l > 0 ? WT[l] : nullptr; b.dZ[l] = dZ[l]; b.part[l] = partial[l];
  }
  if (M == 0) return PPO_OK;
  const dim3 grid(ppo::ceil_div(M, MC_ROWS), towers), block(MC_THREADS);
  hipStream_t st = ppo::as_stream(stream);
#define PPO_CHAIN_FB(ACTV)                                                                              \
  if (va) hipLaunchKernelGGL((mlp_ln_fwd_bwd_kernel<true, ACTV>), grid, block, 0, st, a, hp, b);       \
  else hipLaunchKernelGGL((mlp_ln_fwd_bwd_kernel<false, ACTV>), grid, block, 0, st, a, hp, b);
  switch (act) {
    case ACT_RELU: PPO_CHAIN_FB(ACT_RELU) break;
    case ACT_TANH: PPO_CHAIN_FB(ACT_TANH) break;
    case ACT_SILU: PPO_CHAIN_FB(ACT_SILU) break;
    default: PPO_CHAIN_FB(ACT_NONE) break;
  }
#undef PPO_CHAIN_FB
  return ppo::check_launch(name);
}
