// Pipelined bf16 GEMM instantiated for A stored as fp32, B stored as fp32.
#include "gemm_bf16s.h"

namespace ppo_bf16s {
template <>
int launch_layouts<float, float>(hipStream_t st, const Params& p, int splits, int tile, int a_layout, int b_layout) {
  return launch_layouts_impl<float, float>(st, p, splits, tile, a_layout, b_layout);
}
}  // namespace ppo_bf16s
