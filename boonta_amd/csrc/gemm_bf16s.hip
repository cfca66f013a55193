// Entry points of the pipelined bf16 GEMM (kernel in gemm_bf16s.h), the bf16
// casts and the split-K bf16 epilogue.
#include "gemm_bf16s.h"

namespace {

using namespace ppo_bf16s;

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

__global__ void cast_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
  const int64_t n8 = n / 8;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const floatx4 a = reinterpret_cast<const floatx4*>(x)[2 * i];
    const floatx4 b = reinterpret_cast<const floatx4*>(x)[2 * i + 1];
    uint4 v;
    v.x = pack2(a[0], a[1]);
    v.y = pack2(a[2], a[3]);
    v.z = pack2(b[0], b[1]);
    v.w = pack2(b[2], b[3]);
    reinterpret_cast<uint4*>(y)[i] = v;
  }
  for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = (uint16_t)bf16_bits(x[i]);
}

// Row-pitched cast: y[r][c] = bf16(x[r][c]) for c < cols, 0 for cols <= c < ldy.
// One thread per 8 output elements; rows of x are 16-byte aligned.  IDX:
// the unit index type (32-bit when rows * ldy / 8 fits, which keeps the
// row division short), one unit per thread in that case.
template <typename IDX>
__global__ void cast_bf16_rows_kernel(const float* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y, int64_t ldy,
                                      int rows, int cols) {
  const IDX per_row = (IDX)(ldy / 8);
  const IDX total = (IDX)rows * per_row;
  for (IDX u = (IDX)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (IDX)gridDim.x * blockDim.x) {
    const IDX r = u / per_row;
    const int c = (int)(u - r * per_row) * 8;
    const float* xr = x + (int64_t)r * ldx;
    float v[8];
    if (c + 8 <= cols) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(xr + c);
      const floatx4 b = *reinterpret_cast<const floatx4*>(xr + c + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[e + 4] = b[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (c + e < cols) ? xr[c + e] : 0.f;
    }
    uint4 o;
    o.x = pack2(v[0], v[1]);
    o.y = pack2(v[2], v[3]);
    o.z = pack2(v[4], v[5]);
    o.w = pack2(v[6], v[7]);
    *reinterpret_cast<uint4*>(y + (int64_t)r * ldy + c) = o;
  }
}

// c[r][j] = act(bf16(bf16(sum_s p[s][r][j]) + bf16(bias[j]))), rounded to bf16
// after each step: the epilogue of a split-K bf16 Dense forward.  Partials are
// added in split order.
__global__ void splits_bias_act_bf16_kernel(const float* __restrict__ p, int64_t ldp, int64_t split_stride, int nsplit,
                                            const float* __restrict__ bias, int act, float* __restrict__ c,
                                            int64_t ldc, int rows, int cols) {
  const int64_t total = (int64_t)rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols;
    const int j = (int)(i - r * cols);
    float v = p[r * ldp + j];
    for (int s = 1; s < nsplit; ++s) v += p[s * split_stride + r * ldp + j];
    v = bf16_round(v);
    if (bias) v = bf16_round(v + bf16_round(bias[j]));
    if (act != ACT_NONE) v = bf16_round(ppo::act_fwd(act, v));
    c[r * ldc + j] = v;
  }
}

}  // namespace

// a_bf16 / b_bf16: the operand is stored as bf16 (uint16 bit patterns) rather
// than fp32.
// tile: -1 picks; 0: 256 x 128 (8 waves of 64 x 64), 1: 128 x 128 (4 waves of
// 64 x 64), 2: 256 x 256 (8 waves of 128 x 64; both operands bf16, else 0).
PPO_EXPORT int ppo_gemm_bf16s(void* stream, int a_layout, int b_layout, int a_bf16, int b_bf16, const void* A,
                              int64_t lda, const int32_t* rows, const void* B, int64_t ldb, float* C, int64_t ldc,
                              int M, int N, int K, int splits, int64_t c_split_stride, int epi, const float* bias,
                              int act, int round_out, const float* aux, int64_t ldaux, float* bias_grad, int tile) {
  if (M < 0 || N < 0 || K < 0 || splits < 1 || a_layout < 0 || a_layout > 1 || b_layout < 0 || b_layout > 1 ||
      epi < 0 || epi > 2 || act < 0 || act > 3 || tile > 2)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: bad argument (M=%d N=%d K=%d splits=%d)", M, N, K, splits);
  if (M == 0 || N == 0) return PPO_OK;
  if (!A || !B || !C) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: null operand");
  if (epi == EPI_DACT && !aux) return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: EPI_DACT needs aux");
  if (bias_grad && !(a_layout == 1 && b_layout == 0))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: bias_grad needs a_layout=1, b_layout=0");
  if (splits > 1 && c_split_stride < (int64_t)M * ldc)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: split stride too small");
  // Every load is 16 bytes along the contiguous axis: rows must be 16-byte
  // aligned; an fp32 operand's contiguous extent a multiple of 4; a bf16
  // operand's row pitch at least its extent rounded up to 8 (the tail of a
  // row is read up to that pitch and masked).
  const int a_contig = a_layout == 0 ? K : M;
  const int b_contig = b_layout == 1 ? K : N;
  auto ok = [](const void* ptr, int64_t ld, int contig, int is_bf16) {
    if (!aligned16(ptr)) return false;
    if (is_bf16) return ld % 8 == 0 && ld >= (int64_t)((contig + 7) / 8 * 8);
    return ld % 4 == 0 && contig % 4 == 0;
  };
  if (!ok(A, lda, a_contig, a_bf16) || !ok(B, ldb, b_contig, b_bf16))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gemm_bf16s: operand rows must be 16-byte aligned with 16-byte vector "
                          "extents (lda=%lld ldb=%lld)", (long long)lda, (long long)ldb);
  Params p;
  p.A = A; p.lda = lda; p.rows = rows; p.B = B; p.ldb = ldb; p.C = C; p.ldc = ldc;
  p.c_split_stride = c_split_stride; p.M = M; p.N = N; p.K = K;
  p.k_per_split = ((ppo::ceil_div(K > 0 ? K : 1, splits) + BK - 1) / BK) * BK;
  p.epi = epi; p.bias = bias; p.act = act; p.round_out = round_out; p.aux = aux; p.ldaux = ldaux;
  p.bias_grad = bias_grad;
  if (tile < 0) tile = ((int64_t)ppo::ceil_div(M, 256) * ppo::ceil_div(N, 128) * splits >= 200) ? 0 : 1;
  hipStream_t st = ppo::as_stream(stream);
  if (a_bf16 && b_bf16) return launch_layouts<uint16_t, uint16_t>(st, p, splits, tile, a_layout, b_layout);
  if (a_bf16) return launch_layouts<uint16_t, float>(st, p, splits, tile, a_layout, b_layout);
  if (b_bf16) return launch_layouts<float, uint16_t>(st, p, splits, tile, a_layout, b_layout);
  return launch_layouts<float, float>(st, p, splits, tile, a_layout, b_layout);
}

// y[i] = bf16(x[i]) (round to nearest even), as 16-bit patterns; x, y 16-byte aligned.
PPO_EXPORT int ppo_cast_bf16(void* stream, const float* x, void* y, int64_t n) {
  if (n < 0 || (n > 0 && (!x || !y))) return ppo::set_error(PPO_ERR_ARG, "ppo_cast_bf16: bad argument");
  if (n == 0) return PPO_OK;
  if (!aligned16(x) || !aligned16(y)) return ppo::set_error(PPO_ERR_ARG, "ppo_cast_bf16: buffers must be 16-byte aligned");
  const int64_t blocks = std::min<int64_t>(ppo::ceil_div64(n / 8 + 1, 256), 8192);
  hipLaunchKernelGGL(cast_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, ppo::as_stream(stream), x,
                     static_cast<uint16_t*>(y), n);
  return ppo::check_launch("ppo_cast_bf16");
}

// Row-pitched bf16 copy (the per-update observation copy): y[r][c] = bf16(x[r][c])
// for c < cols and 0 up to ldy (a multiple of 8, >= cols).  x, y 16-byte
// aligned, ldx a multiple of 4.
PPO_EXPORT int ppo_cast_bf16_2d(void* stream, const float* x, int64_t ldx, void* y, int64_t ldy, int rows, int cols) {
  if (rows < 0 || cols < 0 || ldx < cols || ldy % 8 != 0 || ldy < (int64_t)((cols + 7) / 8 * 8) || ldx % 4 != 0)
    return ppo::set_error(PPO_ERR_ARG, "ppo_cast_bf16_2d: bad shape (rows=%d cols=%d ldx=%lld ldy=%lld)", rows, cols,
                          (long long)ldx, (long long)ldy);
  if (rows == 0 || ldy == 0) return PPO_OK;
  if (!x || !y || !aligned16(x) || !aligned16(y))
    return ppo::set_error(PPO_ERR_ARG, "ppo_cast_bf16_2d: buffers must be non-null and 16-byte aligned");
  const int64_t units = (int64_t)rows * (ldy / 8);
  hipStream_t st = ppo::as_stream(stream);
  if (units < ((int64_t)1 << 31) - 256) {
    hipLaunchKernelGGL(cast_bf16_rows_kernel<uint32_t>, dim3((unsigned)ppo::ceil_div64(units, 256)), dim3(256), 0, st,
                       x, ldx, static_cast<uint16_t*>(y), ldy, rows, cols);
  } else {
    const int64_t blocks = std::min<int64_t>(ppo::ceil_div64(units, 256), 16384);
    hipLaunchKernelGGL(cast_bf16_rows_kernel<int64_t>, dim3((unsigned)blocks), dim3(256), 0, st, x, ldx,
                       static_cast<uint16_t*>(y), ldy, rows, cols);
  }
  return ppo::check_launch("ppo_cast_bf16_2d");
}

// Sum of split-K partials with the bf16 Dense epilogue (bias, activation,
// rounding after each step, as ppo_gemm_bf16's epi 1 with round_out).
PPO_EXPORT int ppo_splits_bias_act_bf16(void* stream, const float* partials, int64_t ldp, int64_t split_stride,
                                        int nsplit, const float* bias, int act, float* out, int64_t ldc, int rows,
                                        int cols) {
  if (rows < 0 || cols < 0 || nsplit < 1 || act < 0 || act > 3 || ldp < cols || ldc < cols ||
      (nsplit > 1 && split_stride < (int64_t)rows * ldp))
    return ppo::set_error(PPO_ERR_ARG, "ppo_splits_bias_act_bf16: bad argument (rows=%d cols=%d nsplit=%d)", rows,
                          cols, nsplit);
  if (rows == 0 || cols == 0) return PPO_OK;
  if (!partials || !out) return ppo::set_error(PPO_ERR_ARG, "ppo_splits_bias_act_bf16: null buffer");
  const int64_t blocks = std::min<int64_t>(ppo::ceil_div64((int64_t)rows * cols, 256), 16384);
  hipLaunchKernelGGL(splits_bias_act_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, ppo::as_stream(stream),
                     partials, ldp, split_stride, nsplit, bias, act, out, ldc, rows, cols);
  return ppo::check_launch("ppo_splits_bias_act_bf16");
}
