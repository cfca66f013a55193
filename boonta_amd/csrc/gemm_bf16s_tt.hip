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
