// Linear-recurrence scan h_t = a_t * h_{t-1} + b_t over [batch, steps, features]
// and its vector-Jacobian product, the kernels behind boonta's SSM / MinGRU
// torsos (boonta/networks/kernels/scan.py:13-88: `scan` with its custom VJP;
// the SSM block calls it at networks/blocks/ssm.py:31-55).
//
// Forward:  h_t = a_t h_{t-1} + b_t, h_{-1} = init, accumulated in float32 and
//           stored in the operands' type (float32 or bf16 storage).
// Backward (cotangent g of h):
//           db_t = g_t + a_{t+1} db_{t+1}   (db_{steps-1} = g_{steps-1})
//           da_t = db_t h_{t-1}             (h_{-1} = init)
//           dinit = db_0 a_0
//           with db accumulated in float32 and stored in the operands' type;
//           for bf16 storage da and dinit multiply the stored (rounded) db and
//           are rounded again, as the reference's bf16 array arithmetic does.
//
// The SSM block's episode resets (networks/blocks/ssm.py:45-48) can be folded
// into the same launches (ppo_ssm_scan_*): where done[n, t], the step's decay
// becomes 0 and its input b + a r (r the carry a reset restarts from, zeros
// by default), and the backward carries the reset's own chain rule (da = r db
// there, and no decay into the step).
//
// Layout and parallelism: element (n, t, f) at (n * steps + t) * features + f.
// Each lane owns VW = 4 consecutive features of one sequence where the rows
// allow (one 16-byte float32 or 8-byte bf16 access), so every step reads one
// coalesced row.  When the
// batch x feature lanes alone cannot fill the chip, the time axis is cut into
// C <= 16 chunks, one wave each, in one workgroup: every wave first folds its
// chunk into the affine map (A, B) of h_end = A h_start + B, the waves
// exchange the maps through LDS, and each wave composes the maps before it (in
// time order for the forward, in reverse for the backward) to start its own
// chunk from the exact carry, then re-reads the chunk and writes its outputs.
#include "common.h"

#include <algorithm>

namespace {

constexpr int MAX_CHUNKS = 16;

enum ScanDtype { SCAN_F32 = 0, SCAN_BF16 = 1 };

__device__ __forceinline__ void load_vec(const float* p, int64_t i, float (&v)[1]) { v[0] = p[i]; }
__device__ __forceinline__ void load_vec(const float* p, int64_t i, float (&v)[4]) {
  const floatx4 x = *reinterpret_cast<const floatx4*>(p + i);
  v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
}
__device__ __forceinline__ float bf16_to_f32(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }
__device__ __forceinline__ void load_vec(const uint16_t* p, int64_t i, float (&v)[1]) { v[0] = bf16_to_f32(p[i]); }
__device__ __forceinline__ void load_vec(const uint16_t* p, int64_t i, float (&v)[4]) {
  const uint2 x = *reinterpret_cast<const uint2*>(p + i);
  v[0] = __uint_as_float(x.x << 16); v[1] = __uint_as_float(x.x & 0xffff0000u);
  v[2] = __uint_as_float(x.y << 16); v[3] = __uint_as_float(x.y & 0xffff0000u);
}

__device__ __forceinline__ void store_vec(float* p, int64_t i, const float (&v)[1]) { p[i] = v[0]; }
__device__ __forceinline__ void store_vec(float* p, int64_t i, const float (&v)[4]) {
  floatx4 x;
  x[0] = v[0]; x[1] = v[1]; x[2] = v[2]; x[3] = v[3];
  *reinterpret_cast<floatx4*>(p + i) = x;
}
__device__ __forceinline__ void store_vec(uint16_t* p, int64_t i, const float (&v)[1]) {
  p[i] = (uint16_t)ppo::bf16_bits(v[0]);
}
__device__ __forceinline__ void store_vec(uint16_t* p, int64_t i, const float (&v)[4]) {
  uint2 x;
  x.x = ppo::bf16_bits(v[0]) | (ppo::bf16_bits(v[1]) << 16);
  x.y = ppo::bf16_bits(v[2]) | (ppo::bf16_bits(v[3]) << 16);
  *reinterpret_cast<uint2*>(p + i) = x;
}
// The value a stored element of type S holds (identity for float32).
__device__ __forceinline__ float stored(float x, const float*) { return x; }
__device__ __forceinline__ float stored(float x, const uint16_t*) { return ppo::bf16_round(x); }

struct ScanArgs {
  const void* a;
  const void* b;     // forward: b; backward: the cotangent of h
  const void* h;     // backward: the forward's output
  const void* init;
  void* out;         // forward: h; backward: db
  void* da;
  void* dinit;
  int steps, F, chunk;
  const uint8_t* done;  // [batch, steps] episode starts of the SSM block, or null
  const void* reset;    // [batch, features] carry a done step restarts from, or null (zeros)
};

// The SSM block's reset (networks/blocks/ssm.py:45-48) applied to step t's
// operands: where done, b' = b + a * r and a' = 0, in the storage type's
// arithmetic (each product and sum rounded for bf16).
__device__ __forceinline__ bool is_done(const ScanArgs& p, int64_t n, int t) {
  return p.done && p.done[n * p.steps + t];
}

template <typename S, int VW>
__device__ __forceinline__ void load_reset(const ScanArgs& p, int64_t n, int f0, float (&rv)[VW]) {
  if (p.reset) {
    load_vec(static_cast<const S*>(p.reset), n * (int64_t)p.F + f0, rv);
  } else {
#pragma unroll
    for (int k = 0; k < VW; ++k) rv[k] = 0.f;
  }
}

template <typename S, int VW>
__device__ __forceinline__ void load_ab(const ScanArgs& p, const S* a, const S* b, int64_t base, int64_t n, int t,
                                        int f0, float (&av)[VW], float (&bv)[VW]) {
  load_vec(a, base + (int64_t)t * p.F, av);
  load_vec(b, base + (int64_t)t * p.F, bv);
  if (is_done(p, n, t)) {
    float rv[VW];
    load_reset<S, VW>(p, n, f0, rv);
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      bv[k] = stored(bv[k] + stored(av[k] * rv[k], a), a);
      av[k] = 0.f;
    }
  }
}

// alpha_t = a'_{t+1}, the (reset) decay of the next step; 0 past the last step
template <typename S, int VW>
__device__ __forceinline__ void load_alpha(const ScanArgs& p, const S* a, int64_t base, int64_t n, int t,
                                           float (&al)[VW]) {
  if (t + 1 < p.steps && !is_done(p, n, t + 1)) {
    load_vec(a, base + (int64_t)(t + 1) * p.F, al);
  } else {
#pragma unroll
    for (int k = 0; k < VW; ++k) al[k] = 0.f;
  }
}

// da_t: db'_t h_{t-1} where step t was not reset; r db'_t where it was (the
// cotangent of a through b' = b + a r; a' = 0 passes none)
template <typename S, int VW>
__device__ __forceinline__ void reset_da(const ScanArgs& p, const S* a, int64_t n, int t, int f0,
                                         const float (&dv)[VW], float (&dav)[VW]) {
  if (is_done(p, n, t)) {
    float rv[VW];
    load_reset<S, VW>(p, n, f0, rv);
#pragma unroll
    for (int k = 0; k < VW; ++k) dav[k] = stored(rv[k] * dv[k], a);
  }
}

template <typename S, int VW>
__global__ void __launch_bounds__(64 * MAX_CHUNKS) scan_fwd_kernel(ScanArgs p) {
  // per chunk: the (A, B) maps of its 64 x VW lanes (dynamic: none when C = 1)
  extern __shared__ float smem[];
  float* sA = smem;
  float* sB = smem + (blockDim.x >> 6) * 64 * VW;
  const S* a = static_cast<const S*>(p.a);
  const S* b = static_cast<const S*>(p.b);
  const S* init = static_cast<const S*>(p.init);
  S* out = static_cast<S*>(p.out);
  const int lane = threadIdx.x & 63, c = threadIdx.x >> 6, C = blockDim.x >> 6;
  const int f0 = (blockIdx.x * 64 + lane) * VW;
  const bool ok = f0 < p.F;
  const int64_t n = blockIdx.y;
  const int t0 = c * p.chunk, t1 = min(p.steps, t0 + p.chunk);
  const int64_t base = n * (int64_t)p.steps * p.F + f0;
  float h[VW];
  if (ok) {
    load_vec(init, n * (int64_t)p.F + f0, h);
  } else {
#pragma unroll
    for (int k = 0; k < VW; ++k) h[k] = 0.f;
  }
  if (C > 1) {
    float A[VW], B[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) { A[k] = 1.f; B[k] = 0.f; }
    if (ok) {
#pragma unroll 4
      for (int t = t0; t < t1; ++t) {
        float av[VW], bv[VW];
        load_ab<S, VW>(p, a, b, base, n, t, f0, av, bv);
#pragma unroll
        for (int k = 0; k < VW; ++k) {
          A[k] = av[k] * A[k];
          B[k] = av[k] * B[k] + bv[k];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      sA[(c * 64 + lane) * VW + k] = A[k];
      sB[(c * 64 + lane) * VW + k] = B[k];
    }
    __syncthreads();
    for (int cc = 0; cc < c; ++cc) {
#pragma unroll
      for (int k = 0; k < VW; ++k) h[k] = sA[(cc * 64 + lane) * VW + k] * h[k] + sB[(cc * 64 + lane) * VW + k];
    }
  }
  if (!ok) return;
#pragma unroll 8
  for (int t = t0; t < t1; ++t) {
    float av[VW], bv[VW];
    load_ab<S, VW>(p, a, b, base, n, t, f0, av, bv);
#pragma unroll
    for (int k = 0; k < VW; ++k) h[k] = av[k] * h[k] + bv[k];
    store_vec(out, base + (int64_t)t * p.F, h);
  }
}

template <typename S, int VW>
__global__ void __launch_bounds__(64 * MAX_CHUNKS) scan_bwd_kernel(ScanArgs p) {
  extern __shared__ float smem[];
  float* sA = smem;
  float* sB = smem + (blockDim.x >> 6) * 64 * VW;
  const S* a = static_cast<const S*>(p.a);
  const S* g = static_cast<const S*>(p.b);
  const S* hs = static_cast<const S*>(p.h);
  const S* init = static_cast<const S*>(p.init);
  S* db = static_cast<S*>(p.out);
  S* da = static_cast<S*>(p.da);
  S* dinit = static_cast<S*>(p.dinit);
  const int lane = threadIdx.x & 63, c = threadIdx.x >> 6, C = blockDim.x >> 6;
  const int f0 = (blockIdx.x * 64 + lane) * VW;
  const bool ok = f0 < p.F;
  const int64_t n = blockIdx.y;
  const int t0 = c * p.chunk, t1 = min(p.steps, t0 + p.chunk);
  const int64_t base = n * (int64_t)p.steps * p.F + f0;
  // reverse recurrence d_t = g_t + alpha_t d_{t+1}, alpha_t = a_{t+1}
  // (0 past the last step); d entering this chunk from the chunks after it
  float d[VW];
#pragma unroll
  for (int k = 0; k < VW; ++k) d[k] = 0.f;
  if (C > 1) {
    float P[VW], Q[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) { P[k] = 1.f; Q[k] = 0.f; }
    if (ok) {
#pragma unroll 4
      for (int t = t1 - 1; t >= t0; --t) {
        float al[VW], gv[VW];
        load_alpha<S, VW>(p, a, base, n, t, al);
        load_vec(g, base + (int64_t)t * p.F, gv);
#pragma unroll
        for (int k = 0; k < VW; ++k) {
          P[k] = al[k] * P[k];
          Q[k] = al[k] * Q[k] + gv[k];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      sA[(c * 64 + lane) * VW + k] = P[k];
      sB[(c * 64 + lane) * VW + k] = Q[k];
    }
    __syncthreads();
    for (int cc = C - 1; cc > c; --cc) {
#pragma unroll
      for (int k = 0; k < VW; ++k) d[k] = sA[(cc * 64 + lane) * VW + k] * d[k] + sB[(cc * 64 + lane) * VW + k];
    }
  }
  if (!ok) return;
  // one step of the reverse recurrence; has_next: a_{t+1} exists; first: t = 0
  // (h_{t-1} is init, and dinit is written)
  auto step = [&](int t, bool has_next, bool first) {
    float al[VW], gv[VW], hp[VW];
    if (has_next) {
      load_alpha<S, VW>(p, a, base, n, t, al);
    } else {
#pragma unroll
      for (int k = 0; k < VW; ++k) al[k] = 0.f;
    }
    load_vec(g, base + (int64_t)t * p.F, gv);
    if (first) {
      load_vec(init, n * (int64_t)p.F + f0, hp);
    } else {
      load_vec(hs, base + (int64_t)(t - 1) * p.F, hp);
    }
    float dv[VW], dav[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      d[k] = al[k] * d[k] + gv[k];
      dv[k] = stored(d[k], db);
      dav[k] = dv[k] * hp[k];
    }
    reset_da<S, VW>(p, a, n, t, f0, dv, dav);
    store_vec(db, base + (int64_t)t * p.F, d);
    store_vec(da, base + (int64_t)t * p.F, dav);
    if (first) {
      float a0[VW], di[VW];
      load_vec(a, base, a0);
      if (is_done(p, n, 0)) {
#pragma unroll
        for (int k = 0; k < VW; ++k) a0[k] = 0.f;
      }
#pragma unroll
      for (int k = 0; k < VW; ++k) di[k] = dv[k] * a0[k];
      store_vec(dinit, n * (int64_t)p.F + f0, di);
    }
  };
  // the last and the first step peeled, so the main loop is branch-free and
  // its loads can run ahead of the dependent multiply-adds
  int t = t1 - 1;
  if (t == p.steps - 1) {
    step(t, false, t == 0);
    --t;
  }
  const int lo = max(t0, 1);
#pragma unroll 8
  for (; t >= lo; --t) step(t, true, false);
  if (t == 0 && t >= t0) step(0, true, true);
}

// Register-resident chunks: each wave loads its chunk of at most RL steps once
// (all loads issued before the first multiply-add), folds it into its affine
// map, exchanges the maps through LDS, and writes its outputs from the same
// registers, so chunking costs no second read of the operands.  Steps past
// the chunk's end hold the identity map (a = 1, b = 0 forward; alpha = 1,
// g = 0 backward).
constexpr int RL = 8;

template <typename S, int VW>
__global__ void __launch_bounds__(64 * MAX_CHUNKS) scan_fwd_reg_kernel(ScanArgs p) {
  extern __shared__ float smem[];
  float* sA = smem;
  float* sB = smem + (blockDim.x >> 6) * 64 * VW;
  const S* a = static_cast<const S*>(p.a);
  const S* b = static_cast<const S*>(p.b);
  const S* init = static_cast<const S*>(p.init);
  S* out = static_cast<S*>(p.out);
  const int lane = threadIdx.x & 63, c = threadIdx.x >> 6, C = blockDim.x >> 6;
  const int f0 = (blockIdx.x * 64 + lane) * VW;
  const bool ok = f0 < p.F;
  const int64_t n = blockIdx.y;
  const int t0 = c * RL, t1 = min(p.steps, t0 + RL);
  const int64_t base = n * (int64_t)p.steps * p.F + f0;
  float av[RL][VW], bv[RL][VW], h[VW];
#pragma unroll
  for (int i = 0; i < RL; ++i) {
    if (ok && t0 + i < t1) {
      load_ab<S, VW>(p, a, b, base, n, t0 + i, f0, av[i], bv[i]);
    } else {
#pragma unroll
      for (int k = 0; k < VW; ++k) { av[i][k] = 1.f; bv[i][k] = 0.f; }
    }
  }
  if (ok) {
    load_vec(init, n * (int64_t)p.F + f0, h);
  } else {
#pragma unroll
    for (int k = 0; k < VW; ++k) h[k] = 0.f;
  }
  if (C > 1) {
    float A[VW], B[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) { A[k] = 1.f; B[k] = 0.f; }
#pragma unroll
    for (int i = 0; i < RL; ++i) {
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        A[k] = av[i][k] * A[k];
        B[k] = av[i][k] * B[k] + bv[i][k];
      }
    }
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      sA[(c * 64 + lane) * VW + k] = A[k];
      sB[(c * 64 + lane) * VW + k] = B[k];
    }
    __syncthreads();
    for (int cc = 0; cc < c; ++cc) {
#pragma unroll
      for (int k = 0; k < VW; ++k) h[k] = sA[(cc * 64 + lane) * VW + k] * h[k] + sB[(cc * 64 + lane) * VW + k];
    }
  }
  if (!ok) return;
#pragma unroll
  for (int i = 0; i < RL; ++i) {
#pragma unroll
    for (int k = 0; k < VW; ++k) h[k] = av[i][k] * h[k] + bv[i][k];
    if (t0 + i < t1) store_vec(out, base + (int64_t)(t0 + i) * p.F, h);
  }
}

template <typename S, int VW>
__global__ void __launch_bounds__(64 * MAX_CHUNKS) scan_bwd_reg_kernel(ScanArgs p) {
  extern __shared__ float smem[];
  float* sA = smem;
  float* sB = smem + (blockDim.x >> 6) * 64 * VW;
  const S* a = static_cast<const S*>(p.a);
  const S* g = static_cast<const S*>(p.b);
  const S* hs = static_cast<const S*>(p.h);
  const S* init = static_cast<const S*>(p.init);
  S* db = static_cast<S*>(p.out);
  S* da = static_cast<S*>(p.da);
  S* dinit = static_cast<S*>(p.dinit);
  const int lane = threadIdx.x & 63, c = threadIdx.x >> 6, C = blockDim.x >> 6;
  const int f0 = (blockIdx.x * 64 + lane) * VW;
  const bool ok = f0 < p.F;
  const int64_t n = blockIdx.y;
  const int t0 = c * RL, t1 = min(p.steps, t0 + RL);
  const int64_t base = n * (int64_t)p.steps * p.F + f0;
  // al[i] = a_{t+1} (0 past the last step), gv[i] = g_t, hp[i] = h_{t-1} (init at t = 0)
  float al[RL][VW], gv[RL][VW], hp[RL][VW];
#pragma unroll
  for (int i = 0; i < RL; ++i) {
    const int t = t0 + i;
    if (ok && t < t1) {
      load_alpha<S, VW>(p, a, base, n, t, al[i]);
      load_vec(g, base + (int64_t)t * p.F, gv[i]);
      if (t > 0) {
        load_vec(hs, base + (int64_t)(t - 1) * p.F, hp[i]);
      } else {
        load_vec(init, n * (int64_t)p.F + f0, hp[i]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < VW; ++k) { al[i][k] = 1.f; gv[i][k] = 0.f; hp[i][k] = 0.f; }
    }
  }
  float d[VW];
#pragma unroll
  for (int k = 0; k < VW; ++k) d[k] = 0.f;
  if (C > 1) {
    float P[VW], Q[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) { P[k] = 1.f; Q[k] = 0.f; }
#pragma unroll
    for (int i = RL - 1; i >= 0; --i) {
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        P[k] = al[i][k] * P[k];
        Q[k] = al[i][k] * Q[k] + gv[i][k];
      }
    }
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      sA[(c * 64 + lane) * VW + k] = P[k];
      sB[(c * 64 + lane) * VW + k] = Q[k];
    }
    __syncthreads();
    for (int cc = C - 1; cc > c; --cc) {
#pragma unroll
      for (int k = 0; k < VW; ++k) d[k] = sA[(cc * 64 + lane) * VW + k] * d[k] + sB[(cc * 64 + lane) * VW + k];
    }
  }
  if (!ok) return;
#pragma unroll
  for (int i = RL - 1; i >= 0; --i) {
    const int t = t0 + i;
    float dv[VW], dav[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      d[k] = al[i][k] * d[k] + gv[i][k];
      dv[k] = stored(d[k], db);
      dav[k] = dv[k] * hp[i][k];
    }
    if (t < t1) {
      reset_da<S, VW>(p, a, n, t, f0, dv, dav);
      store_vec(db, base + (int64_t)t * p.F, d);
      store_vec(da, base + (int64_t)t * p.F, dav);
      if (t == 0) {
        float a0[VW], di[VW];
        load_vec(a, base, a0);
        if (is_done(p, n, 0)) {
#pragma unroll
          for (int k = 0; k < VW; ++k) a0[k] = 0.f;
        }
#pragma unroll
        for (int k = 0; k < VW; ++k) di[k] = dv[k] * a0[k];
        store_vec(dinit, n * (int64_t)p.F + f0, di);
      }
    }
  }
}

bool aligned(const void* ptr, int bytes) { return (reinterpret_cast<uintptr_t>(ptr) % bytes) == 0; }

template <typename S, int VW, bool BWD>
int launch(hipStream_t st, const ScanArgs& p, int batch) {
  const int lanes = ppo::ceil_div(p.F, VW);
  const int groups = ppo::ceil_div(lanes, 64);
  const int C = ppo::ceil_div(p.steps, p.chunk);
  dim3 grid(groups, batch), block(64 * C);
  const size_t lds = C > 1 ? 2 * sizeof(float) * (size_t)C * 64 * VW : 0;
  if (BWD) {
    hipLaunchKernelGGL((scan_bwd_kernel<S, VW>), grid, block, lds, st, p);
  } else {
    hipLaunchKernelGGL((scan_fwd_kernel<S, VW>), grid, block, lds, st, p);
  }
  return PPO_OK;
}

template <typename S, int VW, bool BWD>
int launch_reg(hipStream_t st, const ScanArgs& p, int batch) {
  const int groups = ppo::ceil_div(ppo::ceil_div(p.F, VW), 64);
  const int C = ppo::ceil_div(p.steps, RL);
  dim3 grid(groups, batch), block(64 * C);
  const size_t lds = C > 1 ? 2 * sizeof(float) * (size_t)C * 64 * VW : 0;
  if (BWD) {
    hipLaunchKernelGGL((scan_bwd_reg_kernel<S, VW>), grid, block, lds, st, p);
  } else {
    hipLaunchKernelGGL((scan_fwd_reg_kernel<S, VW>), grid, block, lds, st, p);
  }
  return PPO_OK;
}

template <bool BWD>
int dispatch(hipStream_t st, int dtype, ScanArgs p, int batch, const char* what) {
  // 4 features per lane where the rows allow (16-byte float32 or 8-byte bf16
  // accesses; for bf16, 8 per lane would halve the waves in flight).
  // Time chunks re-read their operands, so they are used only when the lanes
  // give too few waves: then enough chunks for twice that, at most 16, each
  // at least 8 steps long.
  const int esize = dtype == SCAN_F32 ? 4 : 2;
  const void* ptrs[8] = {p.a, p.b, p.h, p.init, p.out, p.da, p.dinit, p.reset};
  bool vec = p.F % 4 == 0;
  for (const void* q : ptrs)
    if (q && !aligned(q, 4 * esize)) vec = false;
  const int VW = vec ? 4 : 1;
  const int64_t waves = (int64_t)batch * ppo::ceil_div(ppo::ceil_div(p.F, VW), 64);
  if (p.steps > RL && p.steps <= RL * MAX_CHUNKS) {
    // register-resident chunks of RL steps: no re-read, every load in flight at once
    p.chunk = RL;
    if (dtype == SCAN_F32) {
      if (vec) launch_reg<float, 4, BWD>(st, p, batch); else launch_reg<float, 1, BWD>(st, p, batch);
    } else {
      if (vec) launch_reg<uint16_t, 4, BWD>(st, p, batch); else launch_reg<uint16_t, 1, BWD>(st, p, batch);
    }
    return ppo::check_launch(what);
  }
  // bf16 rows carry half the bytes per load, so bf16 wants more waves in
  // flight before the re-read of a second pass stops paying (measured on
  // [1024, 64, 256]: float32 forward 49 -> 33 us without chunks, bf16 forward
  // 44 -> 34 us with two)
  const int64_t enough = dtype == SCAN_F32 ? 512 : 2048;
  int C = waves >= enough ? 1 : (int)std::min<int64_t>(MAX_CHUNKS, ppo::ceil_div64(2 * enough, waves));
  C = std::max(1, std::min(C, p.steps / 8));
  p.chunk = ppo::ceil_div(p.steps, C);
  if (dtype == SCAN_F32) {
    if (vec) launch<float, 4, BWD>(st, p, batch); else launch<float, 1, BWD>(st, p, batch);
  } else {
    if (vec) launch<uint16_t, 4, BWD>(st, p, batch); else launch<uint16_t, 1, BWD>(st, p, batch);
  }
  return ppo::check_launch(what);
}

}  // namespace

PPO_EXPORT int ppo_linear_scan_fwd(void* stream, int dtype, const void* a, const void* b, const void* init, void* out,
                                   int batch, int steps, int features) {
  if (batch < 0 || steps < 0 || features < 0 || (dtype != SCAN_F32 && dtype != SCAN_BF16))
    return ppo::set_error(PPO_ERR_ARG, "ppo_linear_scan_fwd: bad argument (batch %d steps %d features %d dtype %d)",
                          batch, steps, features, dtype);
  if (batch == 0 || steps == 0 || features == 0) return PPO_OK;
  if (!a || !b || !init || !out) return ppo::set_error(PPO_ERR_ARG, "ppo_linear_scan_fwd: null buffer");
  if (batch > 65535) return ppo::set_error(PPO_ERR_ARG, "ppo_linear_scan_fwd: batch above 65535");
  ScanArgs p{a, b, nullptr, init, out, nullptr, nullptr, steps, features, 0, nullptr, nullptr};
  return dispatch<false>(ppo::as_stream(stream), dtype, p, batch, "ppo_linear_scan_fwd");
}

PPO_EXPORT int ppo_ssm_scan_fwd(void* stream, int dtype, const void* a, const void* b, const uint8_t* done,
                                const void* reset, const void* carry, void* out, int batch, int steps, int features) {
  if (batch < 0 || steps < 0 || features < 0 || (dtype != SCAN_F32 && dtype != SCAN_BF16))
    return ppo::set_error(PPO_ERR_ARG, "ppo_ssm_scan_fwd: bad argument (batch %d steps %d features %d dtype %d)",
                          batch, steps, features, dtype);
  if (batch == 0 || steps == 0 || features == 0) return PPO_OK;
  if (!a || !b || !done || !carry || !out) return ppo::set_error(PPO_ERR_ARG, "ppo_ssm_scan_fwd: null buffer");
  if (batch > 65535) return ppo::set_error(PPO_ERR_ARG, "ppo_ssm_scan_fwd: batch above 65535");
  ScanArgs p{a, b, nullptr, carry, out, nullptr, nullptr, steps, features, 0, done, reset};
  return dispatch<false>(ppo::as_stream(stream), dtype, p, batch, "ppo_ssm_scan_fwd");
}

PPO_EXPORT int ppo_linear_scan_bwd(void* stream, int dtype, const void* a, const void* h, const void* init,
                                   const void* cot, void* da, void* db, void* dinit, int batch, int steps,
                                   int features) {
  if (batch < 0 || steps < 0 || features < 0 || (dtype != SCAN_F32 && dtype != SCAN_BF16))
    return ppo::set_error(PPO_ERR_ARG, "ppo_linear_scan_bwd: bad argument (batch %d steps %d features %d dtype %d)",
                          batch, steps, features, dtype);
  if (batch == 0 || steps == 0 || features == 0) return PPO_OK;
  if (!a || !h || !init || !cot || !da || !db || !dinit)
    return ppo::set_error(PPO_ERR_ARG, "ppo_linear_scan_bwd: null buffer");
  if (batch > 65535) return ppo::set_error(PPO_ERR_ARG, "ppo_linear_scan_bwd: batch above 65535");
  ScanArgs p{a, cot, h, init, db, da, dinit, steps, features, 0, nullptr, nullptr};
  return dispatch<true>(ppo::as_stream(stream), dtype, p, batch, "ppo_linear_scan_bwd");
}

PPO_EXPORT int ppo_ssm_scan_bwd(void* stream, int dtype, const void* a, const void* h, const uint8_t* done,
                                const void* reset, const void* carry, const void* cot, void* da, void* db,
                                void* dcarry, int batch, int steps, int features) {
  if (batch < 0 || steps < 0 || features < 0 || (dtype != SCAN_F32 && dtype != SCAN_BF16))
    return ppo::set_error(PPO_ERR_ARG, "ppo_ssm_scan_bwd: bad argument (batch %d steps %d features %d dtype %d)",
                          batch, steps, features, dtype);
  if (batch == 0 || steps == 0 || features == 0) return PPO_OK;
  if (!a || !h || !done || !carry || !cot || !da || !db || !dcarry)
    return ppo::set_error(PPO_ERR_ARG, "ppo_ssm_scan_bwd: null buffer");
  if (batch > 65535) return ppo::set_error(PPO_ERR_ARG, "ppo_ssm_scan_bwd: batch above 65535");
  ScanArgs p{a, cot, h, carry, db, da, dcarry, steps, features, 0, done, reset};
  return dispatch<true>(ppo::as_stream(stream), dtype, p, batch, "ppo_ssm_scan_bwd");
}
