// Shared pieces of the fp32 GEMM (gemm.hip: register-staged pipeline;
// gemm_f32d.hip: pipeline fed by direct global -> LDS copies): parameters
// and the epilogue.
#pragma once
#include "grad_reduce.h"

namespace ppo_f32 {

enum Epilogue { EPI_STORE = 0, EPI_BIAS_ACT = 1, EPI_DACT = 2 };

struct GemmParams {
  const float* A;
  int64_t lda;
  const int32_t* rows;  // gather indices (A's rows for a_layout 0, reduction rows for 1) or null
  const float* B;
  int64_t ldb;
  float* C;
  int64_t ldc;
  int64_t c_split_stride;  // elements between split-K partial outputs
  int M, N, K;
  int k_per_split;  // multiple of the kernel's stage depth
  int epi;
  const float* bias;  // EPI_BIAS_ACT: [N] or null
  int act;
  float* pre;  // EPI_BIAS_ACT: optional pre-activation output (ldc)
  const float* aux;  // EPI_DACT: activation output (relu, tanh) or input (silu), ld = ldaux
  int64_t ldaux;
  float* bias_grad;  // dW: [splits][N] column sums of B, or null
  // Tower-batched launches (the actor's and critic's same-depth layers in one
  // grid): blockIdx z = tower * splits + split, and tower t's operands sit
  // t * stride elements after tower 0's (rows, the gather, is shared).
  int splits, towers;
  int64_t tA, tB, tC, tBias, tPre, tAux, tBiasGrad;
};

// Up to F32_GROUP_MAX GEMMs of one launch (ppo_gemm_f32_dw_group): problem i
// owns linear tiles [start[i], start[i + 1]) of a gx[i] x gy[i] tile grid per
// split.
constexpr int F32_GROUP_MAX = 8;
struct F32Group {
  GemmParams p[F32_GROUP_MAX];
  int start[F32_GROUP_MAX + 1];
  int gx[F32_GROUP_MAX], gy[F32_GROUP_MAX];
  int count;
};

// The operands of tower t of a tower-batched launch.
__device__ __forceinline__ GemmParams tower_params(const GemmParams& p, int t) {
  GemmParams q = p;
  if (t) {
    q.A += t * p.tA;
    q.B += t * p.tB;
    q.C += t * p.tC;
    if (q.bias) q.bias += t * p.tBias;
    if (q.pre) q.pre += t * p.tPre;
    if (q.aux) q.aux += t * p.tAux;
    if (q.bias_grad) q.bias_grad += t * p.tBiasGrad;
  }
  return q;
}

// Stores a wave's MB x NB blocks of 32 x 32 (v_mfma_f32_32x32x*: lane l holds
// rows 8 (r / 4) + 4 (l / 32) + r % 4 of column l % 32) from row wm0 and column
// wn0 through the epilogue EPI with activation ACT (compile-time, so the
// unrolled element loop holds only their code), and the bias-gradient column
// sums of B.
// PRE: the epilogue's per-lane inputs were loaded earlier by the caller into
// auxv: EPI_DACT's aux values of this lane's outputs (block bi, bj at
// [16 (bi NB + bj) + r]), EPI_BIAS_ACT's bias of block column bj at [bj].
// WT: the outputs are stored device-coherent (write-through past this XCD's
// L2), for a reader in another workgroup of the same launch.
template <bool WT>
__device__ __forceinline__ void store_out(float* q, float v) {
  if constexpr (WT)
    __hip_atomic_store(reinterpret_cast<uint32_t*>(q), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  else
    *q = v;
}

template <int MB, int NB, int EPI, int ACT, bool PRE, bool WT = false>
__device__ __forceinline__ void epilogue_f32_t(const GemmParams& p, floatx16 (&acc)[MB][NB], const float (&bsum)[NB],
                                               bool do_bsum, int wm0, int wn0, int split, int lane,
                                               const float (&auxv)[MB * NB * 16]) {
  const int h = lane >> 5;
  const int l32 = lane & 31;
  float* C = p.C + (int64_t)split * p.c_split_stride;
#pragma unroll
  for (int bi = 0; bi < MB; ++bi) {
#pragma unroll
    for (int bj = 0; bj < NB; ++bj) {
      const int gn = wn0 + bj * 32 + l32;
      const bool n_ok = gn < p.N;
      float bias = 0.f;
      if (EPI == EPI_BIAS_ACT && p.bias && n_ok) bias = PRE ? auxv[bj] : p.bias[gn];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = wm0 + bi * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (!n_ok || gm >= p.M) continue;
        float v = acc[bi][bj][r];
        const int64_t o = (int64_t)gm * p.ldc + gn;
        if (EPI == EPI_BIAS_ACT) {
          v += bias;
          if (p.pre) p.pre[o] = v;
          v = ppo::act_fwd(ACT, v);
        } else if (EPI == EPI_DACT) {
          v *= ppo::act_grad(ACT, PRE ? auxv[16 * (bi * NB + bj) + r] : p.aux[(int64_t)gm * p.ldaux + gn]);
        }
        store_out<WT>(C + o, v);
      }
    }
  }
  if (do_bsum) {
#pragma unroll
    for (int bj = 0; bj < NB; ++bj) {
      const float t = ppo::add_xor32(bsum[bj]);
      const int gn = wn0 + bj * 32 + l32;
      if (h == 0 && gn < p.N) store_out<WT>(p.bias_grad + (int64_t)split * p.N + gn, t);
    }
  }
}

// The epilogue of the launch's kind and activation, chosen once.
// PRE: the bias or the aux values come from auxv (loaded by the caller).
template <int MB, int NB, bool PRE = false>
__device__ __forceinline__ void epilogue_f32(const GemmParams& p, floatx16 (&acc)[MB][NB], const float (&bsum)[NB],
                                             bool do_bsum, int wm0, int wn0, int split, int lane,
                                             const float (&auxv)[MB * NB * 16]) {
#define PPO_EPI_ACTS(E, P)                                                                                  \
  switch (p.act) {                                                                                          \
    case ACT_RELU: epilogue_f32_t<MB, NB, E, ACT_RELU, P>(p, acc, bsum, do_bsum, wm0, wn0, split, lane, auxv); break; \
    case ACT_TANH: epilogue_f32_t<MB, NB, E, ACT_TANH, P>(p, acc, bsum, do_bsum, wm0, wn0, split, lane, auxv); break; \
    case ACT_SILU: epilogue_f32_t<MB, NB, E, ACT_SILU, P>(p, acc, bsum, do_bsum, wm0, wn0, split, lane, auxv); break; \
    default: epilogue_f32_t<MB, NB, E, ACT_NONE, P>(p, acc, bsum, do_bsum, wm0, wn0, split, lane, auxv); break;       \
  }
  if (p.epi == EPI_BIAS_ACT) {
    PPO_EPI_ACTS(EPI_BIAS_ACT, PRE)
  } else if (p.epi == EPI_DACT) {
    PPO_EPI_ACTS(EPI_DACT, PRE)
  } else {
    epilogue_f32_t<MB, NB, EPI_STORE, ACT_NONE, false>(p, acc, bsum, do_bsum, wm0, wn0, split, lane, auxv);
  }
#undef PPO_EPI_ACTS
}

// The copy-fed pipeline (gemm_f32d.hip): 16-byte rows along every operand's
// contiguous axis, stage depth F32D_BK; false when the shape needs the
// register-staged one (a gathered k-outer A with more reduction rows per
// split than the kernel caches).
constexpr int F32D_BK = 32;
constexpr int F32D_KIDX_MAX = 2048;
int launch_dma(hipStream_t st, const GemmParams& p, int splits, int tile, int a_layout, int b_layout);
// A weight-gradient group (A and B k-outer, 64 x 64 copy-fed tiles).
int launch_dw_group(hipStream_t st, const F32Group& g);
// The same with the split-K sums finished in the launch (64 x 64 tiles,
// gathered splits of at most F32D_FINAL_KIDX rows, at most F32D_FINAL_PARTS
// splits of one of the supported counts).
constexpr int F32D_FINAL_KIDX = 512;
constexpr int F32D_FINAL_PARTS = 16;
bool final_parts_supported(int splits);
int launch_dw_group_final(hipStream_t st, const F32Group& g, const ppo_gr::DwFinal& f);

}  // namespace ppo_f32
