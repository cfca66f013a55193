// Shared helpers for the PPO learner kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#ifndef PPO_EXPORT
#define PPO_EXPORT extern "C" __attribute__((visibility("default")))
#endif

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

enum PpoStatus {
  PPO_OK = 0,
  PPO_ERR_ARG = -1,     // invalid argument (shape, pointer, enum)
  PPO_ERR_LAUNCH = -2,  // kernel launch failed
  PPO_ERR_SPACE = -3,   // workspace too small
};

// Activation codes shared with the host side.
enum PpoAct { ACT_NONE = 0, ACT_RELU = 1, ACT_TANH = 2, ACT_SILU = 3 };

namespace ppo {

int set_error(int code, const char* fmt, ...);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(PPO_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return PPO_OK;
}

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Tile coordinates for a GEMM grid (gridDim.x = N tiles, .y = M tiles, .z =
// reduction splits) on a part with 8 XCDs, each with its own L2: the hardware
// hands workgroup w to XCD w % 8, so the linear id is remapped to give XCD x a
// contiguous range of logical tiles, ordered N fastest, then M, then split.
// Tiles that read the same A rows (and, in a split-K launch, the same
// reduction slice) then run together on one XCD and share its L2.
struct TileCoord {
  int n, m, z;
};

__device__ __forceinline__ TileCoord xcd_tile() {
  const int gx = gridDim.x, gy = gridDim.y;
  const int total = gx * gy * gridDim.z;
  const int w = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int x = w & 7, j = w >> 3;
  const int q = total >> 3, r = total & 7;
  const int t = x * q + (x < r ? x : r) + j;
  TileCoord c;
  c.n = t % gx;
  c.m = (t / gx) % gy;
  c.z = t / (gx * gy);
  return c;
}

// Loads that never branch: an out-of-range element reads a clamped, valid
// address and the value is then replaced by zero.  A load under a divergent
// branch makes the compiler wait for it at the branch join; these keep every
// load of a stage in flight together.
__device__ __forceinline__ floatx4 load4_or_zero(const float* p, int64_t i, bool ok) {
  const floatx4 v = *reinterpret_cast<const floatx4*>(p + (ok ? i : 0));
  return ok ? v : floatx4{0.f, 0.f, 0.f, 0.f};
}

__device__ __forceinline__ float load_or_zero(const float* p, int64_t i, bool ok) {
  const float v = p[ok ? i : 0];
  return ok ? v : 0.f;
}

// Round to nearest even bf16 (NaN stays NaN), returned as the fp32 value
// of that bf16 (bits() gives the 16-bit pattern).
// Both results are computed and one is selected: as an if / else the compiler
// makes a divergent branch (exec-mask save / restore) of every rounding in an
// unrolled element loop.
__device__ __forceinline__ uint32_t bf16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;
  return (u & 0x7fffffffu) > 0x7f800000u ? qnan : rne;
}

__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float(bf16_bits(x) << 16); }

// ---- direct global -> LDS copies (global_load_lds_dwordx4) ----
// One 1 KB copy: lane l's 16 bytes at src go to LDS lds_wave_base + 16 l.
// Issued as inline assembly so that the compiler's wait insertion does not
// treat every later LDS read as dependent on it (it cannot tell the slots of
// a ring buffer apart and would wait for all copies); stage_barrier waits
// for the copies explicitly.
__device__ __forceinline__ void lds_copy16(const void* src, void* lds_wave_base) {
  typedef __attribute__((address_space(3))) void lds_void_t;
  const uint32_t m0v = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)(lds_wave_base));
  asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(m0v) : "memory");
}

// Ring-buffer stage barrier: this wave's copies older than the newest N are
// complete and its LDS accesses are done, then every wave of the block meets.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// Stage barrier of a ring whose stages each issue PER_STAGE copies per wave:
// the awaited stage's copies are complete while those of the `younger`
// (<= Y) stages issued after it stay in flight.
template <int PER_STAGE, int Y>
__device__ __forceinline__ void ring_barrier(int younger) {
  if constexpr (Y == 0) {
    stage_barrier<0>();
  } else {
    if (younger >= Y)
      stage_barrier<PER_STAGE * Y>();
    else
      ring_barrier<PER_STAGE, Y - 1>(younger);
  }
}

// XOR applied to the 16-byte chunk index (0..7) of row r of a 128-byte-row
// LDS tile: neither 16-byte copies / stores (8 lanes per row) nor reads of
// one chunk over 32 consecutive rows put two lanes of a bank phase on a bank.
__device__ __forceinline__ int kc_swizzle(int r) {
  return (r & 3) ^ ((r & 4) ? 5 : 0) ^ ((r & 8) ? 3 : 0) ^ ((r & 16) ? 4 : 0);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// The value of lane (l xor M) within each row of 16 lanes (M = 1, 2, 4, 8),
// moved by DPP on the vector ALU instead of an LDS-unit permute
// (__shfl_xor with width 16 compiles to ds_bpermute, a round trip that the
// compiler waits for one at a time).  xor 1 and xor 2 are quad permutes,
// xor 8 is a rotation of the row by 8, xor 4 is the half-row mirror
// (l xor 7) followed by the quad reversal (l xor 3).  Every lane of the row
// must be active.
template <int M>
__device__ __forceinline__ float xor16(float v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "xor16: M in {1, 2, 4, 8}");
  const int x = __float_as_int(v);
  int r;
  if constexpr (M == 1) r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);         // quad_perm [1,0,3,2]
  else if constexpr (M == 2) r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);    // quad_perm [2,3,0,1]
  else if constexpr (M == 4)
    r = __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, true),   // row_half_mirror
                                 0x1B, 0xF, 0xF, true);                                  // quad_perm [3,2,1,0]
  else r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);                           // row_ror:8
  return __int_as_float(r);
}

// x + x[l xor 16] and x + x[l xor 32] for every lane l, from the gfx950
// lane swaps of two copies of x: permlane16_swap exchanges the odd 16-lane
// rows of its first operand with the even rows of its second, permlane32_swap
// the upper half of the first with the lower half of the second, so the two
// results hold x and its partner in every lane (the same sum as
// x + __shfl_xor(x, 16 or 32): the addition is commutative).
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x + x[l xor M] over the whole wave for M = 32, 16, 8, 4, 2, 1 in turn
// (the order of the __shfl_xor loop, so the same bits); every lane active.
__device__ __forceinline__ float wave_sum_lanes(float v) {
  v = add_xor32(v);
  v = add_xor16(v);
  v += xor16<8>(v);
  v += xor16<4>(v);
  v += xor16<2>(v);
  return v + xor16<1>(v);
}

// Sum / max over each row of 16 lanes as the xor butterfly 8, 4, 2, 1 (the
// order of the __shfl_xor loop, so the same bits); every lane gets the result.
__device__ __forceinline__ float sum16(float v) {
  v += xor16<8>(v);
  v += xor16<4>(v);
  v += xor16<2>(v);
  v += xor16<1>(v);
  return v;
}
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, xor16<8>(v));
  v = fmaxf(v, xor16<4>(v));
  v = fmaxf(v, xor16<2>(v));
  v = fmaxf(v, xor16<1>(v));
  return v;
}

// 0 + x[t] + x[t + S] + x[t + 2 S] + ... (i < n) added in that order, with
// the loads of U terms in flight at a time (the order, and so the result,
// of the one-load-per-step loop).
template <int S, int U>
__device__ __forceinline__ double strided_sum_d(const double* __restrict__ x, int n, int t) {
  double acc = 0.0;
  for (int i = t; i < n; i += S * U) {
    double v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = i + S * u;
      v[u] = x[j < n ? j : t];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + S * u < n) acc += v[u];
  }
  return acc;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// LayerNorm arithmetic of the 256-wide fused kernels (Dense + LayerNorm
// forward, the torso chains forward and backward), with every rounding
// step explicit so that kernels compiled apart produce the same bits:
// a row's partial sums (z, then z * z by one fma), its statistics from the
// sums (fast variance, as flax) and the normalised, scaled value.
__device__ __forceinline__ void ln_accum(float z, float& s, float& s2) {
  s += z;
  s2 = __fmaf_rn(z, z, s2);
}
__device__ __forceinline__ void ln_stats256(float s, float s2, float eps, float& mean, float& rstd) {
  mean = s * (1.f / 256.f);
  const float var = fmaxf(__fmaf_rn(-mean, mean, s2 * (1.f / 256.f)), 0.f);
  rstd = rsqrtf(var + eps);
}
__device__ __forceinline__ float ln_apply(float z, float mean, float rstd, float gamma, float beta) {
  return __fmaf_rn(z - mean, rstd * gamma, beta);
}

// LayerNorm of one row held by a wavefront, VPL features per lane (feature
// lane + 64 e in v[e], zeros past the row's F features), with every rounding
// step explicit so that the per-layer LayerNorm kernel and the bf16 chains
// produce the same bits: per-lane sums in e order (z, then z * z by one fma),
// wave sums, mean = s / F, variance max(E[z^2] - mean^2, 0) (flax's fast
// variance), and the normalised, scaled value.
template <int VPL>
__device__ __forceinline__ void ln_row_stats(const float (&v)[VPL], float F, float eps, float& mean, float& rstd) {
  float s = 0.f, s2 = 0.f;
#pragma unroll
  for (int e = 0; e < VPL; ++e) {
    s += v[e];
    s2 = __fmaf_rn(v[e], v[e], s2);
  }
  s = wave_sum(s);
  s2 = wave_sum(s2);
  mean = s / F;
  const float var = fmaxf(__fmaf_rn(-mean, mean, s2 / F), 0.f);
  rstd = rsqrtf(var + eps);
}
// The statistics of R rows at once: per row exactly the operations of
// ln_row_stats (the same sums in the same order, the same butterfly), with
// the rows' reductions interleaved so that their shuffle latencies overlap.
template <int R, int VPL>
__device__ __forceinline__ void ln_rows_stats(const float (&v)[R][VPL], float F, float eps, float (&mean)[R],
                                              float (&rstd)[R]) {
  float s[R], s2[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    s[j] = 0.f;
    s2[j] = 0.f;
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      s[j] += v[j][e];
      s2[j] = __fmaf_rn(v[j][e], v[j][e], s2[j]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
#pragma unroll
    for (int j = 0; j < R; ++j) {
      s[j] += __shfl_xor(s[j], o, 64);
      s2[j] += __shfl_xor(s2[j], o, 64);
    }
#pragma unroll
  for (int j = 0; j < R; ++j) {
    mean[j] = s[j] / F;
    const float var = fmaxf(__fmaf_rn(-mean[j], mean[j], s2[j] / F), 0.f);
    rstd[j] = rsqrtf(var + eps);
  }
}
__device__ __forceinline__ float ln_row_apply(float v, float mean, float rstd, float gamma, float beta) {
  return __fmaf_rn(v - mean, rstd * gamma, beta);
}

// LayerNorm + activation backward of one element of a row, every rounding
// explicit (the per-layer LayerNorm backward and the bf16 chain's give the
// same bits): xh = (z - mean) rstd; the output recomputed as fma(xh, gamma,
// beta), rounded to bf16 when `round` (the bf16 forward rounds it before the
// activation); returns dyl = dy act'(.), the LayerNorm output's cotangent.
// A row's input cotangent is then ln_bwd_dz of its element's g = dyl gamma
// with the row means of g and g xh.
// The kernels that use them compile their LayerNorm backward with
// floating-point contraction off (#pragma clang fp contract(off)): otherwise
// the compiler fuses a product into a later sum (dyl gamma into the row sum
// of g, or into g - mean_g) where it finds it worth it, differently from one
// kernel to another.
template <int ACT>
__device__ __forceinline__ float ln_bwd_dyl(float z, float dy, float mean, float rstd, float gamma, float beta,
                                            bool round, float& xh);
__device__ __forceinline__ float ln_bwd_dz(float g, float xh, float mean_g, float mean_gxh, float rstd) {
#pragma clang fp contract(off)
  return rstd * __fmaf_rn(-xh, mean_gxh, g - mean_g);
}

// x / d for d >= 1 (d may be +inf): the hardware reciprocal (1 ulp) and one
// correction of the quotient from its exact fma residual (Markstein's
// step), instead of the IEEE division sequence, whose scale / fmas / fixup
// steps serialise on VCC and cost about four times as much.  An exact
// product (zero residual) is kept as it is, which keeps the sign of a zero;
// where the residual is not finite (d or x infinite) the product x * (1 / d)
// is the quotient (0, +-inf or NaN as the division gives).  Error bound: with
// a reciprocal within 1 ulp of 1 / d, the quotient q is within about 2 ulp
// and the corrected q1 = q + r (x - d q) within 1 ulp of x / d (faithful);
// Markstein's correct-rounding result needs a correctly rounded reciprocal,
// so correct rounding is not proven here.  Observed: on 6M random SiLU
// arguments it gave the IEEE quotient every time.  Kernels agree with each
// other bit for bit because all of them divide through this function; the
// oracle comparison is to a tolerance.
__device__ __forceinline__ float div_ge1(float x, float d) {
  const float r = __builtin_amdgcn_rcpf(d);
  const float q = x * r;
  const float res = __fmaf_rn(-d, q, x);
  const float q1 = __fmaf_rn(r, res, q);
  return (res == 0.f || !__builtin_isfinite(q1)) ? q : q1;
}

// tanhf out of line: its expansion is long, and kernels that take the
// activation at run time switch on it per element inside unrolled epilogues,
// where every inlined copy (taken or not) would sit between the taken
// case's instructions.
static __device__ __attribute__((noinline)) float tanh_call(float x) { return tanhf(x); }

__device__ __forceinline__ float act_fwd(int act, float x) {
  switch (act) {
    case ACT_RELU: return x > 0.f ? x : 0.f;
    case ACT_TANH: return tanh_call(x);
    case ACT_SILU: return div_ge1(x, 1.f + __expf(-x));
    default: return x;
  }
}

// Derivative of the activation, from its input x (silu) or output y (relu, tanh).
__device__ __forceinline__ float act_grad(int act, float x_or_y) {
  switch (act) {
    case ACT_RELU: return x_or_y > 0.f ? 1.f : 0.f;
    case ACT_TANH: return 1.f - x_or_y * x_or_y;
    case ACT_SILU: {
      float s = div_ge1(1.f, 1.f + __expf(-x_or_y));
      return s * (1.f + x_or_y * (1.f - s));
    }
    default: return 1.f;
  }
}

template <int ACT>
__device__ __forceinline__ float ln_bwd_dyl(float z, float dy, float mean, float rstd, float gamma, float beta,
                                            bool round, float& xh) {
#pragma clang fp contract(off)
  xh = (z - mean) * rstd;
  float yl = __fmaf_rn(xh, gamma, beta);
  if (round) yl = bf16_round(yl);
  const float a = (ACT == ACT_RELU || ACT == ACT_TANH) ? act_fwd(ACT, yl) : yl;
  return dy * act_grad(ACT, a);
}

}  // namespace ppo
