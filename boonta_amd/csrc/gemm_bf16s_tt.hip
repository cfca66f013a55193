// Pipelined bf16 GEMM with both operands stored as bf16: the DMA-fed kernel
// (gemm_bf16d.h), or the register-staged one when a gathered k-outer A
// operand's split holds more reduction rows than the kernel caches.
#include "gemm_bf16d.h"

#ifndef PPO_BF16D_NBUF128
#define PPO_BF16D_NBUF128 2  // ring depth of the 128 x 128 tiles (2 x 32 KB of LDS)
#endif

namespace ppo_bf16s {

template <bool A_K, bool B_K>
int launch_tt(hipStream_t st, const Params& p, int splits, int tile) {
  const bool gathered_k = !A_K && p.rows != nullptr;  // the split's gather indices are cached in LDS
  if (tile == 2 && (!gathered_k || p.k_per_split <= KIDX_256))
    return launch_d<256, 256, 2, 4, A_K, B_K, 2, KIDX_256>(st, p, splits);
  if (gathered_k && p.k_per_split > KIDX_MAX) return launch_tile<A_K, B_K, uint16_t, uint16_t>(st, p, splits, tile);
  if (tile == 1) return launch_d<128, 128, 2, 2, A_K, B_K, PPO_BF16D_NBUF128>(st, p, splits);
  return launch_d<256, 128, 4, 2, A_K, B_K, 3>(st, p, splits);
}

template <>
int launch_layouts<uint16_t, uint16_t>(hipStream_t st, const Params& p, int splits, int tile, int a_layout,
                                       int b_layout) {
  if (a_layout == 0 && b_layout == 0) return launch_tt<true, false>(st, p, splits, tile);
  if (a_layout == 0 && b_layout == 1) return launch_tt<true, true>(st, p, splits, tile);
  if (a_layout == 1 && b_layout == 0) return launch_tt<false, false>(st, p, splits, tile);
  return launch_tt<false, true>(st, p, splits, tile);
}

}  // namespace ppo_bf16s

// Weight gradients of several bf16 Dense layers in one launch (256 x 256
// tiles): problem i is what ppo_gemm_bf16s(a_layout = 1, b_layout = 0,
// a_bf16 = b_bf16 = 1, epi = store, tile = 2) computes from the same
// arguments, with the same bits.
PPO_EXPORT int ppo_gemm_bf16s_dw_group(void* stream, int count, const void* const* A, const int64_t* lda,
                                       const int32_t* const* rows, const void* const* B, const int64_t* ldb,
                                       float* const* C, const int64_t* ldc, const int* M, const int* N, const int* K,
                                       const int* splits, const int64_t* c_split_stride, float* const* bias_grad) {
  using namespace ppo_bf16s;
  if (count < 0 || count > GROUP_MAX || (count > 0 && (!A || !lda || !B || !ldb || !C || !ldc || !M || !N || !K ||
                                                       !splits || !c_split_stride)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s_dw_group: bad argument (count=%d, at most %d)", count,
                          GROUP_MAX);
  GroupParams g = {};
  int total = 0;
  for (int i = 0; i < count; ++i) {
    if (M[i] < 0 || N[i] < 0 || K[i] < 0 || splits[i] < 1)
      return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s_dw_group: problem %d: bad shape (M=%d N=%d K=%d splits=%d)",
                            i, M[i], N[i], K[i], splits[i]);
    if (M[i] == 0 || N[i] == 0) continue;
    if (!A[i] || !B[i] || !C[i]) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s_dw_group: problem %d: null operand", i);
    if (splits[i] > 1 && c_split_stride[i] < (int64_t)M[i] * ldc[i])
      return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s_dw_group: problem %d: split stride too small", i);
    auto ok = [](const void* ptr, int64_t ld, int contig) {
      return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0 && ld % 8 == 0 && ld >= (int64_t)((contig + 7) / 8 * 8);
    };
    if (!ok(A[i], lda[i], M[i]) || !ok(B[i], ldb[i], N[i]) || ldc[i] < N[i])
      return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s_dw_group: problem %d: operand rows must be 16-byte aligned "
                            "with 16-byte vector extents (lda=%lld ldb=%lld ldc=%lld)", i, (long long)lda[i],
                            (long long)ldb[i], (long long)ldc[i]);
    Params& p = g.p[g.count];
    p.A = A[i]; p.lda = lda[i]; p.rows = rows ? rows[i] : nullptr; p.B = B[i]; p.ldb = ldb[i];
    p.C = C[i]; p.ldc = ldc[i]; p.c_split_stride = c_split_stride[i]; p.M = M[i]; p.N = N[i]; p.K = K[i];
    p.k_per_split = ((ppo::ceil_div(K[i] > 0 ? K[i] : 1, splits[i]) + BK - 1) / BK) * BK;
    p.epi = EPI_STORE; p.bias = nullptr; p.act = ACT_NONE; p.round_out = 0; p.aux = nullptr; p.ldaux = 0;
    p.bias_grad = bias_grad ? bias_grad[i] : nullptr;
    if (p.rows && p.k_per_split > KIDX_256)
      return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s_dw_group: problem %d: a gathered split holds %d rows "
                            "(at most %d)", i, p.k_per_split, KIDX_256);
    g.gx[g.count] = ppo::ceil_div(N[i], 256);
    g.gy[g.count] = ppo::ceil_div(M[i], 256);
    g.start[g.count] = total;
    total += g.gx[g.count] * g.gy[g.count] * splits[i];
    ++g.count;
  }
  g.start[g.count] = total;
  if (total == 0) return PPO_OK;
  // 32-deep stages in a four-stage ring (three in flight behind the MFMAs,
  // 128 KB of LDS with the 16 KB gather cache 144 KB: the large-observation
  // update's grouped dW 116 -> 108 us, three stages in flight covering more
  // of the scattered rows' latency; eight 16-deep stages took 119 us); the
  // MFMA sequence along k is that of the 64-deep stages, so the partials are
  // the same bits as tile 2's
  hipLaunchKernelGGL((gemm_bf16d_group_kernel<256, 256, 2, 4, false, false, 4, KIDX_256, 32>), dim3(total), dim3(512),
                     0, ppo::as_stream(stream), g);
  return ppo::check_launch("ppo_gemm_bf16s_dw_group");
}
