// The bf16 torso chain: the 512-wide Dense -> LayerNorm -> activation layers
// of a bf16 network (flax Dense and LayerNorm with a bf16 compute dtype and
// fp32 parameters, as the large-observation workload composes them;
// boonta/networks/network.py:38-49) after the first layer's contraction, in
// one launch.
//
// The first Dense contracts the bf16 observation rows on the split-K GEMM and
// leaves split partials; this launch takes them from there.  A workgroup owns
// 32 rows and runs them through every remaining step: the split sum with the
// first Dense's bias, its LayerNorm + activation, then each later layer's
// 512 x 512 contraction on bf16 MFMA (v_mfma_f32_32x32x16_bf16), its bias,
// LayerNorm and activation, the layer's output staying in LDS as the next
// layer's input.  Only what the backward and the heads read goes to HBM:
// each layer's pre-LayerNorm Z (fp32), mean, rstd and the bf16 output Y16
// (the next weight gradient's operand), and the last layer's fp32 output.
//
// Rounding follows the per-layer launches step for step, so the chain is
// bit-identical to them: the split sum in split order, rounded to bf16, plus
// the bf16-rounded bias, rounded again (splits_bias_act_bf16); an
// accumulator rounded to bf16, plus the rounded bias, rounded (the bf16
// GEMM's bias epilogue); each contraction is the same MFMA sequence as the
// GEMM's (k ascending in steps of 16, one accumulator, the same operand
// placement); the LayerNorm statistics and output are ppo::ln_row_stats /
// ln_row_apply, which the per-layer LayerNorm kernel also uses, with the
// features of a row in the same lanes (feature lane + 64 e).
//
// Kernel operands come from a packed image (ppo_pack_bf16_operands) in which
// each 1 KB chunk is one wave's MFMA B operand for one 32-column block and
// one 16-deep k step, so every operand load is a coalesced 16 bytes per lane
// straight into registers, several k steps ahead of the MFMAs.  The workgroup's
// eight waves own 64 output columns each; no kernel data goes through LDS.
#include "common.h"

namespace {

constexpr int C16_F = 512;                 // features in and out of every chain layer
constexpr int C16_ROWS = 32;               // rows per workgroup
constexpr int C16_WAVES = 8;               // two per SIMD: one's LayerNorm latencies hide behind the other's work
constexpr int C16_THREADS = 64 * C16_WAVES;
constexpr int C16_CPW = C16_F / C16_WAVES;  // output columns per wave in a contraction
constexpr int C16_BJ = C16_CPW / 32;        // its 32-column MFMA blocks
constexpr int C16_MAXL = 8;
constexpr int C16_KSTEPS = C16_F / 16;     // 16-deep k steps of one contraction
constexpr int C16_NB = C16_F / 32;         // 32-column blocks of one layer
constexpr int A_PITCH = C16_F + 8;         // bf16 per LDS activation row: rows 16 bytes apart in bank order
constexpr int Z_PITCH = C16_F + 8;         // floats per LDS pre-activation row: rows 4 apart 32 banks apart
constexpr int PF = 8;                      // k steps of kernel operands in flight per wave
constexpr int VPL = C16_F / 64;            // features per lane in the LayerNorm stage
static_assert(C16_KSTEPS % PF == 0, "the operand ring must divide the k steps");

// ------------------------------------------------------------ operand packing
// Packed MFMA B-operand image of a contraction out[m][n] = sum_k A[m][k] B[k][n]
// with B [KD][ND]: chunk c = kb * (ND / 32) + nb (1 KB) holds, for lane l and
// element i, B[16 kb + 8 (l >> 5) + i][32 nb + (l & 31)] at 512 c + 8 l + i.
// fwd: B = W (a layer's kernel [K][N], row pitch ldw); bwd: B = W^T (the input
// cotangent dZ W^T contracts over the output features).
struct PackArgs {  // slot l: one kernel (the chain's layers, then a head)
  const uint16_t* W[C16_MAXL + 1];
  uint16_t* fwd[C16_MAXL + 1];
  uint16_t* bwd[C16_MAXL + 1];
  int64_t ldw[C16_MAXL + 1];
  int K[C16_MAXL + 1], N[C16_MAXL + 1];
  int nvalid[C16_MAXL + 1];  // kernel columns present: forward columns and backward k rows nvalid .. N - 1 pack as zeros
};

__global__ void __launch_bounds__(256) pack_operands_kernel(PackArgs a) {
  const int l = blockIdx.y;
  const bool bwd = blockIdx.z != 0;
  uint16_t* dst = bwd ? a.bwd[l] : a.fwd[l];
  const uint16_t* W = a.W[l];
  if (!dst || !W) return;
  const int K = a.K[l], N = a.N[l], nvalid = a.nvalid[l];
  const int64_t ldw = a.ldw[l];
  const int KD = bwd ? N : K, ND = bwd ? K : N;
  const int64_t units = (int64_t)KD * ND / 8;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(u & 63);
    const int64_t c = u >> 6;
    const int nb = (int)(c % (ND / 32)), kb = (int)(c / (ND / 32));
    const int k0 = 16 * kb + 8 * (lane >> 5), n = 32 * nb + (lane & 31);
    uint16_t v[8];
    if (bwd && nvalid == N && ldw % 8 == 0) {
      // B[k][n] = W[n][k]: eight consecutive k of kernel row n
      const uint4 q = *reinterpret_cast<const uint4*>(W + (int64_t)n * ldw + k0);
      *reinterpret_cast<uint4*>(v) = q;
    } else if (bwd) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = k0 + i < nvalid ? W[(int64_t)n * ldw + k0 + i] : (uint16_t)0;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = n < nvalid ? W[(int64_t)(k0 + i) * ldw + n] : (uint16_t)0;
    }
    *reinterpret_cast<uint4*>(dst + 8 * u) = *reinterpret_cast<const uint4*>(v);
  }
}

// ------------------------------------------------------------- forward chain
struct Fwd16Args {
  const float* part;  // the first Dense's split partials [nsplit][M] (row pitch ldp, split stride pstride)
  int64_t ldp, pstride;
  int nsplit, M, L;
  float eps;
  int64_t ld;                        // row pitch of Z, Y and Y16
  int z16;                           // Z[l] holds bf16 (the pre-activations are bf16 numbers), else fp32
  const uint16_t* Wp[C16_MAXL];      // layer l >= 1: packed forward operand image of its kernel
  const float* bias[C16_MAXL];       // may be null
  const float* gamma[C16_MAXL];
  const float* beta[C16_MAXL];
  float* Z[C16_MAXL];
  float* Y[C16_MAXL];                // may be null (only the bf16 output is read)
  uint16_t* Y16[C16_MAXL];
  float* mean[C16_MAXL];
  float* rstd[C16_MAXL];
  // optional: a Dense head on the last layer's output (nh <= 256 outputs):
  // its packed forward operand image (512 x 32 ceil(nh / 32)), bias, and the
  // rounded head outputs [M][ldh]
  const uint16_t* Wh;
  const float* bh;
  float* head;
  int64_t ldh;
  int nh;
};

template <int ACT>
__global__ void __launch_bounds__(C16_THREADS, 1) mlp16_ln_fwd_kernel(Fwd16Args a) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[C16_ROWS * A_PITCH];
  __shared__ __attribute__((aligned(16))) float sZ[C16_ROWS * Z_PITCH];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m0 = blockIdx.x * C16_ROWS;
  const int h = lane >> 5, l32 = lane & 31;
  constexpr int RPW = C16_ROWS / C16_WAVES;  // rows of a wave's row stages
  const int r0 = RPW * wave;         // the wave's first row in the tile

  // kernel operand ring: w[s % PF][j] holds k step s of column block C16_BJ wave + j
  bf16x8 w[PF][C16_BJ];
  auto load_w = [&](int l, int s, bf16x8 (&dst)[C16_BJ]) {
    const uint16_t* Ws = a.Wp[l] + ((int64_t)s * C16_NB + C16_BJ * wave) * 512 + 8 * lane;
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j) dst[j] = *reinterpret_cast<const bf16x8*>(Ws + 512 * j);
  };
  float g[VPL], be[VPL];
  auto load_ln = [&](int l) {
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      g[e] = a.gamma[l][lane + 64 * e];
      be[e] = a.beta[l][lane + 64 * e];
    }
  };
  // The wave's rows r0 .. r0 + 7 of a 32 x 512 fp32 LDS tile to global rows,
  // 16 bytes per lane (chunk c: row c / 128, features 4 (c % 128) ..).
  auto rows_out_f32 = [&](float* dst, const float* tile) {
#pragma unroll
    for (int i = 0; i < RPW * C16_F / 256; ++i) {
      const int c = 64 * i + lane, rr = c >> 7, c4 = c & 127;
      const int grow = m0 + r0 + rr;
      const floatx4 v = *reinterpret_cast<const floatx4*>(tile + (r0 + rr) * Z_PITCH + 4 * c4);
      if (grow < a.M) *reinterpret_cast<floatx4*>(dst + (int64_t)grow * a.ld + 4 * c4) = v;
    }
  };
  // The same rows as bf16 (values that are bf16 numbers), 16 bytes per lane.
  auto rows_out_bf16 = [&](uint16_t* dst, const float* tile) {
#pragma unroll
    for (int i = 0; i < RPW * C16_F / 512; ++i) {
      const int c = 64 * i + lane, rr = c >> 6, c8 = c & 63;
      const int grow = m0 + r0 + rr;
      const floatx4 u = *reinterpret_cast<const floatx4*>(tile + (r0 + rr) * Z_PITCH + 8 * c8);
      const floatx4 v = *reinterpret_cast<const floatx4*>(tile + (r0 + rr) * Z_PITCH + 8 * c8 + 4);
      uint4 q;
      q.x = ppo::bf16_bits(u[0]) | (ppo::bf16_bits(u[1]) << 16);
      q.y = ppo::bf16_bits(u[2]) | (ppo::bf16_bits(u[3]) << 16);
      q.z = ppo::bf16_bits(v[0]) | (ppo::bf16_bits(v[1]) << 16);
      q.w = ppo::bf16_bits(v[2]) | (ppo::bf16_bits(v[3]) << 16);
      if (grow < a.M) *reinterpret_cast<uint4*>(dst + (int64_t)grow * a.ld + 8 * c8) = q;
    }
  };
  // LayerNorm + activation of the wave's rows from their pre-activations in
  // sZ (feature lane + 64 e in lane), as the per-layer LayerNorm kernel's bf16
  // path: the result rounded to bf16, the activation, rounded again unless it
  // is ReLU.  The bf16 output goes to sA (the next layer's input) and, 16
  // bytes per lane, to Y16; the fp32 output (where Y[l] is set) through sZ
  // to Y; mean and rstd from lanes 0 .. 7.
  auto ln_rows = [&](int l) {
    float v[RPW][VPL];
#pragma unroll
    for (int j = 0; j < RPW; ++j)
#pragma unroll
      for (int e = 0; e < VPL; ++e) v[j][e] = sZ[(r0 + j) * Z_PITCH + lane + 64 * e];
    float mean[RPW], rstd[RPW];
    ppo::ln_rows_stats<RPW, VPL>(v, (float)C16_F, a.eps, mean, rstd);
    float* Yl = a.Y[l];
#pragma unroll
    for (int j = 0; j < RPW; ++j)
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        float o = ppo::bf16_round(ppo::ln_row_apply(v[j][e], mean[j], rstd[j], g[e], be[e]));
        o = ppo::act_fwd(ACT, o);
        if (ACT != ACT_RELU && ACT != ACT_NONE) o = ppo::bf16_round(o);
        sA[(r0 + j) * A_PITCH + lane + 64 * e] = (uint16_t)ppo::bf16_bits(o);
        if (Yl) sZ[(r0 + j) * Z_PITCH + lane + 64 * e] = o;
      }
    uint16_t* Y16 = a.Y16[l];
#pragma unroll
    for (int i = 0; i < RPW * C16_F / 512; ++i) {
      const int c = 64 * i + lane, rr = c >> 6, c8 = c & 63;
      const int grow = m0 + r0 + rr;
      const uint4 q = *reinterpret_cast<const uint4*>(sA + (r0 + rr) * A_PITCH + 8 * c8);
      if (grow < a.M) *reinterpret_cast<uint4*>(Y16 + (int64_t)grow * a.ld + 8 * c8) = q;
    }
    if (Yl) rows_out_f32(Yl, sZ);
    float mv = mean[0], rv = rstd[0];
#pragma unroll
    for (int j = 1; j < RPW; ++j) {
      mv = lane == j ? mean[j] : mv;
      rv = lane == j ? rstd[j] : rv;
    }
    if (lane < RPW && m0 + r0 + lane < a.M) {
      a.mean[l][m0 + r0 + lane] = mv;
      a.rstd[l][m0 + r0 + lane] = rv;
    }
  };

  // layer 0: split sum + bias (the first Dense's epilogue) of the wave's
  // rows, 16 bytes per lane: to Z and to the wave's rows of sZ; then its
  // LayerNorm.  The partials and parameters are loaded before any store.
  {
    load_ln(0);
    const float* bias = a.bias[0];
    floatx4 b4[2];
#pragma unroll
    for (int q = 0; q < 2; ++q)
      b4[q] = bias ? *reinterpret_cast<const floatx4*>(bias + 4 * (64 * q + lane)) : floatx4{0.f, 0.f, 0.f, 0.f};
    if (a.L > 1) {
#pragma unroll
      for (int s = 0; s < PF; ++s) load_w(1, s, w[s]);
    }
    constexpr int NC = RPW * C16_F / 256;  // 16-byte chunks per lane
    constexpr int NB = NC > 8 ? 2 : 1;     // batches of them
#pragma unroll
    for (int hb = 0; hb < NB; ++hb) {
      floatx4 p[NC / NB];
      const float* src[NC / NB];
#pragma unroll
      for (int ii = 0; ii < NC / NB; ++ii) {
        const int c = 64 * (hb * (NC / NB) + ii) + lane, rr = c >> 7, c4 = c & 127;
        const int grow = m0 + r0 + rr;
        src[ii] = a.part + (int64_t)(grow < a.M ? grow : a.M - 1) * a.ldp + 4 * c4;
        p[ii] = *reinterpret_cast<const floatx4*>(src[ii]);
      }
      for (int sp = 1; sp < a.nsplit; ++sp)
#pragma unroll
        for (int ii = 0; ii < NC / NB; ++ii) p[ii] += *reinterpret_cast<const floatx4*>(src[ii] + sp * a.pstride);
#pragma unroll
      for (int ii = 0; ii < NC / NB; ++ii) {
        const int i = hb * (NC / NB) + ii;
        const int c = 64 * i + lane, rr = c >> 7, c4 = c & 127;
        const floatx4 bq = b4[i & 1];
        floatx4 v;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[k] = ppo::bf16_round(p[ii][k]);
          if (bias) v[k] = ppo::bf16_round(v[k] + ppo::bf16_round(bq[k]));
        }
        const int grow = m0 + r0 + rr;
        *reinterpret_cast<floatx4*>(sZ + (r0 + rr) * Z_PITCH + 4 * c4) = v;
        if (grow < a.M) {
          if (a.z16) {
            uint2 q;
            q.x = ppo::bf16_bits(v[0]) | (ppo::bf16_bits(v[1]) << 16);
            q.y = ppo::bf16_bits(v[2]) | (ppo::bf16_bits(v[3]) << 16);
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.Z[0]) + (int64_t)grow * a.ld + 4 * c4) = q;
          } else {
            *reinterpret_cast<floatx4*>(a.Z[0] + (int64_t)grow * a.ld + 4 * c4) = v;
          }
        }
      }
    }
    ln_rows(0);
  }

  for (int l = 1; l < a.L; ++l) {
    // the layer's parameters, ahead of the contraction (its loads are waited
    // for with the kernel operands', none after a store)
    const float* bias = a.bias[l];
    float bc[C16_BJ];
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j) bc[j] = bias ? bias[C16_CPW * wave + 32 * j + l32] : 0.f;
    load_ln(l);
    __syncthreads();  // the layer input is in sA
    floatx16 acc[C16_BJ];
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
    const uint16_t* arow = sA + l32 * A_PITCH + 8 * h;
    bf16x8 x8[2];
    x8[0] = *reinterpret_cast<const bf16x8*>(arow);
#pragma unroll
    for (int s = 0; s < C16_KSTEPS; ++s) {
      if (s + 1 < C16_KSTEPS) x8[(s + 1) & 1] = *reinterpret_cast<const bf16x8*>(arow + 16 * (s + 1));
#pragma unroll
      for (int j = 0; j < C16_BJ; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x8[s & 1], w[s % PF][j], acc[j], 0, 0, 0);
      // refill the slot just consumed: step s + PF of this layer, or the
      // next layer's first steps (in flight across the epilogue)
      if (s + PF < C16_KSTEPS)
        load_w(l, s + PF, w[s % PF]);
      else if (l + 1 < a.L)
        load_w(l + 1, s + PF - C16_KSTEPS, w[s % PF]);
      // keep each step's refill where it is: the scheduler would otherwise
      // sink the loads towards their use and shorten the prefetch distance
      __builtin_amdgcn_sched_barrier(0);
    }
    // bias epilogue of the contraction into the pre-activation tile
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j) {
      const int n = C16_CPW * wave + 32 * j + l32;
      const float bb = ppo::bf16_round(bc[j]);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * h + (r & 3);
        float v = ppo::bf16_round(acc[j][r]);
        if (bias) v = ppo::bf16_round(v + bb);
        sZ[row * Z_PITCH + n] = v;
      }
    }
    __syncthreads();  // every wave's columns are in sZ; sA is free
    if (a.z16)
      rows_out_bf16(reinterpret_cast<uint16_t*>(a.Z[l]), sZ);
    else
      rows_out_f32(a.Z[l], sZ);
    ln_rows(l);
  }

  // the head: wave j < ceil(nh / 32) computes output columns 32 j .. 32 j + 31
  // of the tile's 32 rows from the last layer's bf16 output, as the bf16
  // GEMM's bias epilogue rounds them (the same MFMA sequence: k ascending in
  // steps of 16, one accumulator)
  if (a.Wh) {
    __syncthreads();  // the last layer's output of every row is in sA
    const int nhb = (a.nh + 31) / 32;
    if (wave < nhb) {
      constexpr int HPF = 8;
      const uint16_t* Wj = a.Wh + (int64_t)wave * 512 + 8 * lane;
      const int64_t step = (int64_t)nhb * 512;
      bf16x8 hw[HPF];
#pragma unroll
      for (int s = 0; s < HPF; ++s) hw[s] = *reinterpret_cast<const bf16x8*>(Wj + s * step);
      const int n = 32 * wave + l32;
      // the bias goes out with the first kernel chunks, not after the last MFMA
      const float bh = a.bh ? a.bh[n < a.nh ? n : a.nh - 1] : 0.f;
      floatx16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
      const uint16_t* arow = sA + l32 * A_PITCH + 8 * h;
#pragma unroll
      for (int s = 0; s < C16_KSTEPS; ++s) {
        const bf16x8 x8 = *reinterpret_cast<const bf16x8*>(arow + 16 * s);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x8, hw[s % HPF], acc, 0, 0, 0);
        if (s + HPF < C16_KSTEPS) hw[s % HPF] = *reinterpret_cast<const bf16x8*>(Wj + (s + HPF) * step);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (n < a.nh) {
        const float bb = ppo::bf16_round(bh);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int grow = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
          float v = ppo::bf16_round(acc[r]);
          if (a.bh) v = ppo::bf16_round(v + bb);
          if (grow < a.M) a.head[(int64_t)grow * a.ldh + n] = v;
        }
      }
    }
  }
}

// ------------------------------------------------------------ backward chain
struct Bwd16Args {
  const float* dY;  // cotangent of the top layer's output [M] (row pitch lddy)
  int64_t lddy;
  int M, L;
  int64_t ld;                        // row pitch of Z and dZ16
  int z16;                           // Z[l] holds bf16, else fp32
  const uint16_t* Wb[C16_MAXL];      // layer l >= 1: packed backward operand image of its kernel
  const float* Z[C16_MAXL];
  const float* mean[C16_MAXL];
  const float* rstd[C16_MAXL];
  const float* gamma[C16_MAXL];
  const float* beta[C16_MAXL];
  uint16_t* dZ16[C16_MAXL];
  float* part[C16_MAXL];             // [blocks][2 * 512]: scale | bias gradient sums of each workgroup's rows
  // optional: the top cotangent from a Dense head's output cotangents dhead
  // [M][lddh] (nh columns) and the head kernel's packed backward operand
  // image Whb (W^T over nhk 16-deep k steps); dY is then not read
  const float* dhead;
  int64_t lddh;
  const uint16_t* Whb;
  int nh, nhk;
  // optional with the head: the rounded cotangents as bf16 [M][ld16] (zero
  // past nh), the B operand of the head's weight gradient
  uint16_t* dhead16;
  int64_t ld16;
};

// From the top layer down: the LayerNorm + activation backward of layer l
// (bf16 forward: the recomputed output rounded before the activation) gives
// dZ_l, rounded to bf16 (dZ16, the weight gradient's operand) and the scale
// and bias gradient sums of the workgroup's 32 rows; below the top, the
// input cotangent dY_{l-1} = dZ16_l W_l^T (bf16 MFMA over the packed
// backward operand image, k = the layer's outputs ascending in steps of 16,
// rounded to bf16 as the bf16 GEMM's epilogue) stays in LDS for layer l - 1.
// dZ16 of a row is bit-identical to the per-layer launches'
// (ppo_layernorm_act_bwd_bf16_out16, ppo_gemm_bf16s); the gradient sums
// follow this launch's own row blocks.
template <int ACT>
__global__ void __launch_bounds__(C16_THREADS, 1) mlp16_ln_bwd_kernel(Bwd16Args a) {
#pragma clang fp contract(off)  // the LayerNorm backward's roundings as written (as the per-layer kernel)
  __shared__ __attribute__((aligned(16))) uint16_t sA[C16_ROWS * A_PITCH];  // dZ16 tile
  __shared__ __attribute__((aligned(16))) float sD[C16_ROWS * Z_PITCH];     // dY tile
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = blockIdx.x * C16_ROWS;
  const int h = lane >> 5, l32 = lane & 31;
  constexpr int RPW = C16_ROWS / C16_WAVES;
  constexpr int RB = RPW;  // rows per LayerNorm batch
  const int r0 = RPW * wave;
  // the wave's gradient-sum slot (4 KB) lies in its own rows of sD, free once
  // the wave has read its cotangents
  static_assert(RPW * Z_PITCH >= 2 * C16_F, "a wave's rows of sD hold its gradient sums");
  float* red = sD + r0 * Z_PITCH;

  bf16x8 w[PF][C16_BJ];
  auto load_w = [&](int l, int s, bf16x8 (&dst)[C16_BJ]) {
    const uint16_t* Ws = a.Wb[l] + ((int64_t)s * C16_NB + C16_BJ * wave) * 512 + 8 * lane;
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j) dst[j] = *reinterpret_cast<const bf16x8*>(Ws + 512 * j);
  };
  // layer l's pre-activations and statistics of the wave's rows (lane + 64 e)
  float zv[RPW][VPL], mu[RPW], rs[RPW];
  auto load_z = [&](int l) {
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int grow = m0 + r0 + j;
      const int64_t gc = grow < a.M ? grow : a.M - 1;
      mu[j] = a.mean[l][gc];
      rs[j] = a.rstd[l][gc];
      if (a.z16) {
        const uint16_t* z = reinterpret_cast<const uint16_t*>(a.Z[l]) + gc * a.ld + lane;
#pragma unroll
        for (int e = 0; e < VPL; ++e) zv[j][e] = __uint_as_float((uint32_t)z[64 * e] << 16);
      } else {
#pragma unroll
        for (int e = 0; e < VPL; ++e) zv[j][e] = a.Z[l][gc * a.ld + lane + 64 * e];
      }
    }
  };

  load_z(a.L - 1);
  if (a.L > 1) {
#pragma unroll
    for (int s = 0; s < PF; ++s) load_w(a.L - 1, s, w[s]);
  }
  if (a.Whb) {
    // the top cotangent from the head: dY = dhead W^T, the head's output
    // cotangents rounded to bf16 as the bf16 GEMM stages them (sA row r,
    // columns k < 16 nhk, zero past nh), then its MFMA sequence (k ascending
    // in steps of 16) and its rounding
    for (int i = threadIdx.x; i < C16_ROWS * 16 * a.nhk; i += C16_THREADS) {
      const int r = i / (16 * a.nhk), k = i % (16 * a.nhk);
      const int grow = m0 + r;
      const float v = (k < a.nh && grow < a.M) ? a.dhead[(int64_t)grow * a.lddh + k] : 0.f;
      const uint16_t bits = (uint16_t)ppo::bf16_bits(v);
      sA[r * A_PITCH + k] = bits;
      if (a.dhead16 && grow < a.M && k < a.ld16) a.dhead16[(int64_t)grow * a.ld16 + k] = bits;
    }
    __syncthreads();
    floatx16 acc[C16_BJ];
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
    const uint16_t* arow = sA + l32 * A_PITCH + 8 * h;
    for (int s = 0; s < a.nhk; ++s) {
      const bf16x8 x8 = *reinterpret_cast<const bf16x8*>(arow + 16 * s);
      const uint16_t* Ws = a.Whb + ((int64_t)s * C16_NB + C16_BJ * wave) * 512 + 8 * lane;
#pragma unroll
      for (int j = 0; j < C16_BJ; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x8, *reinterpret_cast<const bf16x8*>(Ws + 512 * j), acc[j],
                                                         0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j) {
      const int n = C16_CPW * wave + 32 * j + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) sD[(8 * (r >> 2) + 4 * h + (r & 3)) * Z_PITCH + n] = ppo::bf16_round(acc[j][r]);
    }
    __syncthreads();  // every row's cotangent is in sD; sA is free
  } else {
    // the top cotangent: the wave's rows into sD, 16 bytes per lane
#pragma unroll
    for (int i = 0; i < RPW * C16_F / 256; ++i) {
      const int c = 64 * i + lane, rr = c >> 7, c4 = c & 127;
      const int grow = m0 + r0 + rr;
      const floatx4 v =
          *reinterpret_cast<const floatx4*>(a.dY + (int64_t)(grow < a.M ? grow : a.M - 1) * a.lddy + 4 * c4);
      *reinterpret_cast<floatx4*>(sD + (r0 + rr) * Z_PITCH + 4 * c4) = v;
    }
  }

  for (int l = a.L - 1; l >= 0; --l) {
    float g[VPL], be[VPL], ag[VPL], ab[VPL];
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      g[e] = a.gamma[l][lane + 64 * e];
      be[e] = a.beta[l][lane + 64 * e];
      ag[e] = 0.f;
      ab[e] = 0.f;
    }
#pragma unroll
    for (int hb = 0; hb < RPW / RB; ++hb) {
      float xh[RB][VPL], gg[RB][VPL], sg[RB], sgx[RB];
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const int jj = hb * RB + j;
        const bool live = m0 + r0 + jj < a.M;
        sg[j] = 0.f;
        sgx[j] = 0.f;
#pragma unroll
        for (int e = 0; e < VPL; ++e) {
          const float dv = sD[(r0 + jj) * Z_PITCH + lane + 64 * e];
          const float dyl = ppo::ln_bwd_dyl<ACT>(zv[jj][e], dv, mu[jj], rs[jj], g[e], be[e], true, xh[j][e]);
          if (live) {
            ag[e] = __fmaf_rn(dyl, xh[j][e], ag[e]);
            ab[e] += dyl;
          }
          gg[j][e] = dyl * g[e];
          sg[j] += gg[j][e];
          sgx[j] = __fmaf_rn(gg[j][e], xh[j][e], sgx[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        sg[j] = ppo::wave_sum_lanes(sg[j]);
        sgx[j] = ppo::wave_sum_lanes(sgx[j]);
      }
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const int jj = hb * RB + j;
        const float mg = sg[j] / (float)C16_F, mgx = sgx[j] / (float)C16_F;
#pragma unroll
        for (int e = 0; e < VPL; ++e)
          sA[(r0 + jj) * A_PITCH + lane + 64 * e] =
              (uint16_t)ppo::bf16_bits(ppo::ln_bwd_dz(gg[j][e], xh[j][e], mg, mgx, rs[jj]));
      }
    }
    // dZ16 of the wave's rows, 16 bytes per lane
    uint16_t* dZ = a.dZ16[l];
#pragma unroll
    for (int i = 0; i < RPW * C16_F / 512; ++i) {
      const int c = 64 * i + lane, rr = c >> 6, c8 = c & 63;
      const int grow = m0 + r0 + rr;
      const uint4 q = *reinterpret_cast<const uint4*>(sA + (r0 + rr) * A_PITCH + 8 * c8);
      if (grow < a.M) *reinterpret_cast<uint4*>(dZ + (int64_t)grow * a.ld + 8 * c8) = q;
    }
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      red[lane + 64 * e] = ag[e];
      red[C16_F + lane + 64 * e] = ab[e];
    }
    __syncthreads();  // dZ16 of every row in sA; every wave's sums in its slot
    {
      float* part = a.part[l] + (int64_t)blockIdx.x * 2 * C16_F;
#pragma unroll
      for (int k = 0; k < 2 * C16_F / C16_THREADS; ++k) {
        const int f = tid + C16_THREADS * k;
        float t = 0.f;
#pragma unroll
        for (int wv = 0; wv < C16_WAVES; ++wv) t += sD[RPW * wv * Z_PITCH + f];
        part[f] = t;
      }
    }
    if (l == 0) break;
    __syncthreads();  // the sums are read before the contraction's epilogue overwrites sD
    floatx16 acc[C16_BJ];
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
    const uint16_t* arow = sA + l32 * A_PITCH + 8 * h;
    bf16x8 x8[2];
    x8[0] = *reinterpret_cast<const bf16x8*>(arow);
#pragma unroll
    for (int s = 0; s < C16_KSTEPS; ++s) {
      if (s + 1 < C16_KSTEPS) x8[(s + 1) & 1] = *reinterpret_cast<const bf16x8*>(arow + 16 * (s + 1));
#pragma unroll
      for (int j = 0; j < C16_BJ; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x8[s & 1], w[s % PF][j], acc[j], 0, 0, 0);
      if (s + PF < C16_KSTEPS)
        load_w(l, s + PF, w[s % PF]);
      else if (l - 1 >= 1)
        load_w(l - 1, s + PF - C16_KSTEPS, w[s % PF]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // the next layer's pre-activations, in flight across the epilogue
    load_z(l - 1);
#pragma unroll
    for (int j = 0; j < C16_BJ; ++j) {
      const int n = C16_CPW * wave + 32 * j + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * h + (r & 3);
        sD[row * Z_PITCH + n] = ppo::bf16_round(acc[j][r]);
      }
    }
    __syncthreads();  // dY_{l-1} of every row in sD; sA is free
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

PPO_EXPORT int ppo_mlp16_max_layers() { return C16_MAXL; }

// Packs the bf16 kernels W[l] [K][N] (row pitch ldw) of L layers into the
// MFMA operand images the bf16 chains read: fwd[l] for the forward's
// contraction over K, bwd[l] for the input cotangent's contraction over N
// (each K * N bf16; a null W[l], or a null output, is skipped).  With Wh
// non-null the same launch also packs a head kernel Wh [K][nh] (row pitch
// ldwh) as ppo_pack_bf16_operand_padded would, into fwdh and bwdh.
PPO_EXPORT int ppo_pack_bf16_operands(void* stream, int L, const void* const* W, int64_t ldw, int K, int N,
                                      void* const* fwd, void* const* bwd, const void* Wh, int64_t ldwh, int nh,
                                      int nh_pad, void* fwdh, void* bwdh) {
  if (L < 1 || L > C16_MAXL || K < 16 || N < 32 || K % 32 || N % 32 || ldw < N || ldw % 8 || !W)
    return ppo::set_error(PPO_ERR_ARG, "ppo_pack_bf16_operands: bad argument (L=%d K=%d N=%d ldw=%lld)", L, K, N,
                          (long long)ldw);
  if (Wh && (!fwdh || nh < 1 || ldwh < nh || nh_pad < nh || nh_pad % 32 || !aligned16(fwdh) ||
             (bwdh && !aligned16(bwdh))))
    return ppo::set_error(PPO_ERR_ARG, "ppo_pack_bf16_operands: bad head (nh=%d nh_pad=%d)", nh, nh_pad);
  PackArgs a{};
  for (int l = 0; l < L; ++l) {
    a.ldw[l] = ldw; a.K[l] = K; a.N[l] = N; a.nvalid[l] = N;
    a.W[l] = static_cast<const uint16_t*>(W[l]);
    a.fwd[l] = fwd ? static_cast<uint16_t*>(fwd[l]) : nullptr;
    a.bwd[l] = bwd ? static_cast<uint16_t*>(bwd[l]) : nullptr;
    if ((a.W[l] && !aligned16(a.W[l])) || (a.fwd[l] && !aligned16(a.fwd[l])) || (a.bwd[l] && !aligned16(a.bwd[l])))
      return ppo::set_error(PPO_ERR_ARG, "ppo_pack_bf16_operands: layer %d needs 16-byte aligned buffers", l);
  }
  int slots = L;
  if (Wh) {  // the head rides in one more slot of the same launch
    a.ldw[L] = ldwh; a.K[L] = K; a.N[L] = nh_pad; a.nvalid[L] = nh;
    a.W[L] = static_cast<const uint16_t*>(Wh);
    a.fwd[L] = static_cast<uint16_t*>(fwdh);
    a.bwd[L] = static_cast<uint16_t*>(bwdh);
    slots = L + 1;
  }
  const int64_t units = (int64_t)K * N / 8;
  const dim3 grid((unsigned)std::min<int64_t>(ppo::ceil_div64(units, 256), 1024), slots, 2);
  hipLaunchKernelGGL(pack_operands_kernel, grid, dim3(256), 0, ppo::as_stream(stream), a);
  return ppo::check_launch("ppo_pack_bf16_operands");
}

// Packs one bf16 kernel W [K][N] (row pitch ldw) as the operand images of a
// head narrower than a 32-column MFMA block, padded with zeros to n_pad (a
// multiple of 32 >= N): fwd, the forward operand of the K x n_pad
// contraction; bwd (may be null), W^T as the operand of the input
// cotangent's contraction over the n_pad outputs.
PPO_EXPORT int ppo_pack_bf16_operand_padded(void* stream, const void* W, int64_t ldw, int K, int N, int n_pad,
                                            void* fwd, void* bwd) {
  if (!W || !fwd || K < 16 || K % 32 || N < 1 || ldw < N || n_pad < N || n_pad % 32 || !aligned16(fwd) ||
      (bwd && !aligned16(bwd)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_pack_bf16_operand_padded: bad argument (K=%d N=%d n_pad=%d)", K, N,
                          n_pad);
  PackArgs a{};
  a.ldw[0] = ldw; a.K[0] = K; a.N[0] = n_pad; a.nvalid[0] = N;
  a.W[0] = static_cast<const uint16_t*>(W);
  a.fwd[0] = static_cast<uint16_t*>(fwd);
  a.bwd[0] = static_cast<uint16_t*>(bwd);
  const int64_t units = (int64_t)K * n_pad / 8;
  const dim3 grid((unsigned)std::min<int64_t>(ppo::ceil_div64(units, 256), 1024), 1, 2);
  hipLaunchKernelGGL(pack_operands_kernel, grid, dim3(256), 0, ppo::as_stream(stream), a);
  return ppo::check_launch("ppo_pack_bf16_operand_padded");
}

// Forward of the bf16 chain on M rows from the first Dense's split
// partials: layer 0's split sum, bias, LayerNorm and activation, then layers
// 1 .. L-1 (512 x 512 kernels, packed forward operands Wp[l]), each with its
// bias, LayerNorm and activation.  Writes Z, Y16, mean, rstd of every layer
// and Y where Y[l] is non-null (Z as bf16 when z16: its values are bf16
// numbers); with Wh non-null also the head on the last
// layer's output (nh outputs, Wh its packed forward operand image of
// 32 ceil(nh / 32) columns, bias bh) into head [M][ldh].
PPO_EXPORT int ppo_mlp16_ln_fwd(void* stream, int L, const float* part, int64_t ldp, int64_t part_stride,
                                int nsplit, int M, const void* const* Wp, const float* const* bias,
                                const float* const* gamma, const float* const* beta, float* const* Z,
                                float* const* Y, void* const* Y16, int64_t ld, float* const* mean,
                                float* const* rstd, float eps, int act, const void* Wh, const float* bh, int nh,
                                float* head, int64_t ldh, int z16) {
  if (Wh && (nh < 1 || nh > 32 * C16_WAVES || !head || ldh < nh || !aligned16(Wh)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_mlp16_ln_fwd: bad head (nh=%d ldh=%lld)", nh, (long long)ldh);
  if (L < 1 || L > C16_MAXL || M < 0 || nsplit < 1 || act < 0 || act > 3 || !part || !aligned16(part) ||
      ldp < C16_F || ldp % 4 || (nsplit > 1 && (part_stride < (int64_t)M * ldp || part_stride % 4)) ||
      ld < C16_F || ld % 8 || !gamma || !beta || !Z || !Y16 || !mean || !rstd || !bias || (L > 1 && !Wp))
    return ppo::set_error(PPO_ERR_ARG, "ppo_mlp16_ln_fwd: bad argument (L=%d M=%d nsplit=%d)", L, M, nsplit);
  if (M == 0) return PPO_OK;
  Fwd16Args a{};
  a.part = part; a.ldp = ldp; a.pstride = part_stride; a.nsplit = nsplit; a.M = M; a.L = L; a.eps = eps;
  a.ld = ld; a.z16 = z16 != 0;
  a.Wh = static_cast<const uint16_t*>(Wh); a.bh = bh; a.head = head; a.ldh = ldh; a.nh = nh;
  for (int l = 0; l < L; ++l) {
    if (!gamma[l] || !beta[l] || !Z[l] || !Y16[l] || !mean[l] || !rstd[l] || !aligned16(Z[l]) ||
        !aligned16(Y16[l]) || (Y && Y[l] && !aligned16(Y[l])) || (bias[l] && !aligned16(bias[l])) ||
        (l > 0 && (!Wp[l] || !aligned16(Wp[l]))))
      return ppo::set_error(PPO_ERR_ARG, "ppo_mlp16_ln_fwd: layer %d: missing or unaligned buffer", l);
    a.Wp[l] = l > 0 ? static_cast<const uint16_t*>(Wp[l]) : nullptr;
    a.bias[l] = bias[l]; a.gamma[l] = gamma[l]; a.beta[l] = beta[l];
    a.Z[l] = Z[l]; a.Y[l] = Y ? Y[l] : nullptr; a.Y16[l] = static_cast<uint16_t*>(Y16[l]);
    a.mean[l] = mean[l]; a.rstd[l] = rstd[l];
  }
  const dim3 grid(ppo::ceil_div(M, C16_ROWS)), block(C16_THREADS);
  hipStream_t st = ppo::as_stream(stream);
  switch (act) {
    case ACT_RELU: hipLaunchKernelGGL(mlp16_ln_fwd_kernel<ACT_RELU>, grid, block, 0, st, a); break;
    case ACT_TANH: hipLaunchKernelGGL(mlp16_ln_fwd_kernel<ACT_TANH>, grid, block, 0, st, a); break;
    case ACT_SILU: hipLaunchKernelGGL(mlp16_ln_fwd_kernel<ACT_SILU>, grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL(mlp16_ln_fwd_kernel<ACT_NONE>, grid, block, 0, st, a); break;
  }
  return ppo::check_launch("ppo_mlp16_ln_fwd");
}

PPO_EXPORT int ppo_mlp16_ln_bwd_blocks(int rows) { return rows > 0 ? ppo::ceil_div(rows, C16_ROWS) : 0; }

// Backward of the bf16 chain on M rows from dY, the cotangent of the top
// layer's output (fp32, row pitch lddy): per layer from the top, dZ16[l]
// (bf16, row pitch ld) and part[l] ([ppo_mlp16_ln_bwd_blocks(M)][2 * 512]:
// the LayerNorm scale | bias gradient sums of each 32-row block), and below
// the top the input cotangent through Wb[l], the packed backward operand
// image of layer l's kernel.  With Whb non-null the top cotangent is instead
// dhead W_h^T from the head's output cotangents dhead [M][lddh] (nh columns)
// and Whb, the head kernel's packed backward image over nh_pad (32 or 64)
// outputs (ppo_pack_bf16_operand_padded), as the bf16 head GEMM rounds it.
// z16: Z[l] holds the forward's bf16 Z.  dhead16 (with the head; may be
// null): receives the rounded head cotangents as bf16 [M][lddh16], zero in
// columns nh .. lddh16 - 1 (lddh16 a multiple of 8, nh <= lddh16 <= nh_pad).
PPO_EXPORT int ppo_mlp16_ln_bwd(void* stream, int L, const float* dY, int64_t lddy, int M, const void* const* Wb,
                                const float* const* Z, const float* const* mean, const float* const* rstd,
                                const float* const* gamma, const float* const* beta, void* const* dZ16, int64_t ld,
                                float* const* part, int act, const float* dhead, int64_t lddh, const void* Whb,
                                int nh, int nh_pad, int z16, void* dhead16, int64_t lddh16) {
  if (Whb && (!dhead || nh < 1 || lddh < nh || nh_pad < nh || nh_pad % 32 || nh_pad > 64 || !aligned16(Whb)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_mlp16_ln_bwd: bad head (nh=%d nh_pad=%d)", nh, nh_pad);
  if (dhead16 && (!Whb || lddh16 < nh || lddh16 > nh_pad || lddh16 % 8 || !aligned16(dhead16)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_mlp16_ln_bwd: bad bf16 head cotangent (lddh16=%lld nh=%d nh_pad=%d)",
                          (long long)lddh16, nh, nh_pad);
  if (L < 1 || L > C16_MAXL || M < 0 || act < 0 || act > 3 || (!Whb && (!dY || !aligned16(dY) || lddy < C16_F ||
      lddy % 4)) || ld < C16_F || ld % 8 || !Z || !mean || !rstd || !gamma || !beta || !dZ16 || !part ||
      (L > 1 && !Wb))
    return ppo::set_error(PPO_ERR_ARG, "ppo_mlp16_ln_bwd: bad argument (L=%d M=%d)", L, M);
  if (M == 0) return PPO_OK;
  Bwd16Args a{};
  a.dY = dY; a.lddy = lddy; a.M = M; a.L = L; a.ld = ld; a.z16 = z16 != 0;
  a.dhead = dhead; a.lddh = lddh; a.Whb = static_cast<const uint16_t*>(Whb); a.nh = nh; a.nhk = nh_pad / 16;
  a.dhead16 = static_cast<uint16_t*>(dhead16); a.ld16 = lddh16;
  for (int l = 0; l < L; ++l) {
    if (!Z[l] || !mean[l] || !rstd[l] || !gamma[l] || !beta[l] || !dZ16[l] || !part[l] || !aligned16(dZ16[l]) ||
        (l > 0 && (!Wb[l] || !aligned16(Wb[l]))))
      return ppo::set_error(PPO_ERR_ARG, "ppo_mlp16_ln_bwd: layer %d: missing or unaligned buffer", l);
    a.Wb[l] = l > 0 ? static_cast<const uint16_t*>(Wb[l]) : nullptr;
    a.Z[l] = Z[l]; a.mean[l] = mean[l]; a.rstd[l] = rstd[l]; a.gamma[l] = gamma[l]; a.beta[l] = beta[l];
    a.dZ16[l] = static_cast<uint16_t*>(dZ16[l]); a.part[l] = part[l];
  }
  const dim3 grid(ppo::ceil_div(M, C16_ROWS)), block(C16_THREADS);
  hipStream_t st = ppo::as_stream(stream);
  switch (act) {
    case ACT_RELU: hipLaunchKernelGGL(mlp16_ln_bwd_kernel<ACT_RELU>, grid, block, 0, st, a); break;
    case ACT_TANH: hipLaunchKernelGGL(mlp16_ln_bwd_kernel<ACT_TANH>, grid, block, 0, st, a); break;
    case ACT_SILU: hipLaunchKernelGGL(mlp16_ln_bwd_kernel<ACT_SILU>, grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL(mlp16_ln_bwd_kernel<ACT_NONE>, grid, block, 0, st, a); break;
  }
  return ppo::check_launch("ppo_mlp16_ln_bwd");
}
