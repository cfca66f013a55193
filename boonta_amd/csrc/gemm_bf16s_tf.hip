// Pipelined bf16 GEMM instantiated for A stored as bf16, B stored as fp32.
#include "gemm_bf16s.h"

namespace ppo_bf16s {
template <>
int launch_layouts<uint16_t, float>(hipStream_t st, const Params& p, int splits, int tile, int a_layout, int b_layout) {
  return launch_layouts_impl<uint16_t, float>(st, p, splits, tile, a_layout, b_layout);
}
}  // namespace ppo_bf16s
