// GRU recurrence of the recurrent learner (flax.linen.GRUCell inside boonta's
// RNN block, boonta/networks/blocks/rnn.py:34-54), one kernel launch per time
// step, forward and backward through time.
//
// Per step t, for sequence b and hidden unit u (flax GRUCell, flax 0.12.8):
//   hp  = done_t[b] ? 0 : h_{t-1}                       reset_carry, rnn.py:11-16,42-45
//   r   = sigmoid(xr + hp Whr)     z = sigmoid(xz + hp Whz)
//   hn  = hp Whn + bhn             n = tanh(xn + r * hn)
//   h_t = (1 - z) * n + z * hp
// where xr/xz/xn = x Wi* + bi* come precomputed for all steps from one large
// GEMM over the whole sequence minibatch.
//
// Layouts (row-major, explicit leading dimensions):
//   xi     [Bm, 3H]  columns [xn | xr | xz]
//   wh     [H, 3H]   columns [r | z | n]       (the three flax kernels side by side)
//   gates  [Bm, 4H]  columns [n | r | z | hn]  (saved for the backward)
//   dgate  [Bm, 4H]  columns [dan | dar | daz | dhn]
// so that dgate[:, 0:3H] is the cotangent of xi (the input projections) and
// dgate[:, H:4H] is the cotangent of hp Wh (the recurrent projections).
//
// Work split: a workgroup of 4 wave64s owns 16 sequences x 16 hidden units.
// The contraction is split across the 4 waves (each a quarter of K) on
// v_mfma_f32_16x16x4f32; the partial tiles meet in LDS and one thread per
// (sequence, unit) finishes the gate arithmetic.  The forward step computes
// the r, z and n columns of its units together so the gates never leave the
// workgroup.  The backward step at t contracts dgate_t[:, H:4H] with Wh^T for
// its units, adds the direct path dh_t * z_t, applies the reset of step t and
// the head cotangent of step t-1, then produces dgate_{t-1} for its units:
// one launch per step in both directions, no inter-workgroup synchronisation.
#include "common.h"

namespace {

constexpr int TILE = 16;
constexpr int WAVES = 4;

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }

// Branches only on which flag arrays exist (uniform), never on loaded data,
// so the flag loads stay in flight with the others.
__device__ __forceinline__ bool done_at(const uint8_t* term, const uint8_t* trunc, const int32_t* rows,
                                        int b) {
  if (!term && !trunc) return false;
  const int64_t i = rows ? (int64_t)rows[b] : (int64_t)b;
  const uint32_t t1 = term ? term[i] : 0u;
  const uint32_t t2 = trunc ? trunc[i] : 0u;
  return (t1 | t2) != 0u;
}

// Scheduling barrier: the batch of independent loads above it is issued
// before the first MFMA below it consumes one of them.
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

struct FwdArgs {
  const float* xi; int64_t ldxi;
  const float* hprev; int64_t ldh; const int32_t* hprev_rows;
  const uint8_t* term; const uint8_t* trunc; const int32_t* flag_rows;
  const float* wh; int64_t ldwh;
  const float* bhn;
  float* h_out; int64_t ldo;
  float* hp_out; int64_t ldhp;
  float* gates; int64_t ldg;
  int Bm, H;
};

// grid (ceil(Bm / 16), H / 16), block 256.  NIT: 16-wide k steps per wave
// (H / 64) when known at compile time (all of a wave's loads then issue
// before its first MFMA); 0: a runtime loop.  The epilogue's operands are
// loaded at entry, so their latency overlaps the contraction's.
template <int NIT>
__global__ void __launch_bounds__(256) gru_fwd_step_kernel(FwdArgs a) {
  __shared__ float red[WAVES][3][TILE][TILE + 1];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int b0 = blockIdx.x * TILE;
  const int u0 = blockIdx.y * TILE;
  const int H = a.H;

  // A operand: row i = lane % 16 of the tile, k = base + 4 * (lane / 16) + s.
  const int i = lane & 15;
  const int kq = lane >> 4;
  const int b = b0 + i;
  const bool b_ok = b < a.Bm;
  const int bc = b_ok ? b : b0;
  const int64_t ra = a.hprev_rows ? (int64_t)a.hprev_rows[bc] : (int64_t)bc;
  const float* hrow = a.hprev + ra * a.ldh;
  const int kspan = H / WAVES;
  const int kbeg = wave * kspan;
  const float* wcol = a.wh + u0 + i;  // B operand: column u0 + i of each gate block
  auto load = [&](int base, floatx4& av, float (&bv)[3][4]) {
    const int k = base + 4 * kq;
    av = *reinterpret_cast<const floatx4*>(hrow + k);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float* wr = wcol + (int64_t)(k + s) * a.ldwh;
#pragma unroll
      for (int g = 0; g < 3; ++g) bv[g][s] = wr[g * H];
    }
  };
  floatx4 av[NIT > 0 ? NIT : 1];
  float bv[NIT > 0 ? NIT : 1][3][4];
  if (NIT > 0) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) load(kbeg + 16 * it, av[it], bv[it]);
  }
  const bool live = b_ok && !done_at(a.term, a.trunc, a.flag_rows, b);

  // epilogue operands of this thread's (sequence, unit)
  const int ti = tid >> 4;   // sequence within the tile
  const int tj = tid & 15;   // unit within the tile
  const int bb = b0 + ti;
  const int u = u0 + tj;
  const bool bb_ok = bb < a.Bm;
  const int bbc = bb_ok ? bb : b0;
  const float* x = a.xi + (int64_t)bbc * a.ldxi;
  const float xn = x[u], xr = x[H + u], xz = x[2 * H + u];
  const float bhn = a.bhn[u];
  const bool reset_e = bb_ok ? done_at(a.term, a.trunc, a.flag_rows, bb) : true;
  const int64_t re = a.hprev_rows ? (int64_t)a.hprev_rows[bbc] : (int64_t)bbc;
  const float hp_raw = a.hprev[re * a.ldh + u];
  issue_fence();

  floatx4 acc[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) acc[g] = floatx4{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](floatx4 avv, const float (&bvv)[3][4]) {
    if (!live) avv = floatx4{0.f, 0.f, 0.f, 0.f};  // a reset sequence starts from h = 0
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int g = 0; g < 3; ++g) acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(avv[s], bvv[g][s], acc[g], 0, 0, 0);
    }
  };
  if (NIT > 0) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) mma(av[it], bv[it]);
  } else {
    for (int base = kbeg; base < kbeg + kspan; base += 16) {
      floatx4 a1;
      float b1[3][4];
      load(base, a1, b1);
      mma(a1, b1);
    }
  }
  // D layout: lane holds rows 4 * (lane / 16) + v, column lane % 16.
#pragma unroll
  for (int g = 0; g < 3; ++g)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][g][4 * kq + v][i] = acc[g][v];
  __syncthreads();

  if (!bb_ok) return;
  float ar = 0.f, az = 0.f, an = 0.f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    ar += red[w][0][ti][tj];
    az += red[w][1][ti][tj];
    an += red[w][2][ti][tj];
  }
  const float hp = reset_e ? 0.f : hp_raw;
  const float r = sigmoidf_(xr + ar);
  const float z = sigmoidf_(xz + az);
  const float hn = an + bhn;
  const float n = tanhf(xn + r * hn);
  const float h = (1.f - z) * n + z * hp;
  a.h_out[(int64_t)bb * a.ldo + u] = h;
  if (a.hp_out) a.hp_out[(int64_t)bb * a.ldhp + u] = hp;
  if (a.gates) {
    float* g = a.gates + (int64_t)bb * a.ldg;
    g[u] = n;
    g[H + u] = r;
    g[2 * H + u] = z;
    g[3 * H + u] = hn;
  }
}

struct BwdArgs {
  // the contraction at step t (dg == null: first call, no step t)
  const float* dg; int64_t lddg;         // dgate_t[:, H:4H]
  const float* wh; int64_t ldwh;
  const float* dh_t; int64_t lddht;
  const float* z_t; int64_t ldz;          // gates_t + 2H
  const uint8_t* term; const uint8_t* trunc; const int32_t* flag_rows;  // resets of step t
  // step s = t - 1
  const float* dout; int64_t lddo;        // head cotangent of h_s
  const float* gates_s; int64_t ldg;
  const float* hp_s; int64_t ldhp;
  float* dh_s; int64_t lddhs;
  float* dgate_s; int64_t lddgs;
  int Bm, H;
};

// grid (ceil(Bm / 16), H / 16), block 256.  NIT: 16-wide k steps per wave
// (3H / 64) when known at compile time; 0: a runtime loop.  The epilogue's
// operands are loaded at entry.
template <int NIT>
__global__ void __launch_bounds__(256) gru_bwd_step_kernel(BwdArgs a) {
  __shared__ float red[WAVES][TILE][TILE + 1];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int b0 = blockIdx.x * TILE;
  const int u0 = blockIdx.y * TILE;
  const int H = a.H;
  const int ti = tid >> 4;
  const int tj = tid & 15;
  const int bb = b0 + ti;
  const int u = u0 + tj;
  const bool bb_ok = bb < a.Bm;
  const int bbc = bb_ok ? bb : b0;

  // contraction operands: dhp[b][u] = sum_c dgate_t[b][H + c] * Wh[u][c], c < 3H
  const int i = lane & 15;
  const int kq = lane >> 4;
  const bool live = b0 + i < a.Bm;
  const float* arow = a.dg ? a.dg + (int64_t)(live ? b0 + i : b0) * a.lddg : nullptr;
  const float* brow = a.wh ? a.wh + (int64_t)(u0 + i) * a.ldwh : nullptr;
  const int kspan = 3 * H / WAVES;
  const int kbeg = wave * kspan;
  floatx4 av[NIT > 0 ? NIT : 1], bv[NIT > 0 ? NIT : 1];
  if (NIT > 0 && a.dg) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int k = kbeg + 16 * it + 4 * kq;
      av[it] = *reinterpret_cast<const floatx4*>(arow + k);
      bv[it] = *reinterpret_cast<const floatx4*>(brow + k);
    }
  }
  // epilogue operands
  float dh = a.dout[(int64_t)bbc * a.lddo + u];
  const float* gs = a.gates_s + (int64_t)bbc * a.ldg;
  const float n = gs[u], r = gs[H + u], z = gs[2 * H + u], hn = gs[3 * H + u];
  const float hp = a.hp_s[(int64_t)bbc * a.ldhp + u];
  float direct = 0.f;
  bool reset_t = false;
  if (a.dg) {
    direct = a.dh_t[(int64_t)bbc * a.lddht + u] * a.z_t[(int64_t)bbc * a.ldz + u];
    reset_t = done_at(a.term, a.trunc, a.flag_rows, bbc);
  }
  issue_fence();

  if (a.dg) {
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](floatx4 x, floatx4 y) {
      if (!live) x = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[s], y[s], acc, 0, 0, 0);
    };
    if (NIT > 0) {
#pragma unroll
      for (int it = 0; it < NIT; ++it) mma(av[it], bv[it]);
    } else {
      for (int base = kbeg; base < kbeg + kspan; base += 16) {
        const int k = base + 4 * kq;
        mma(*reinterpret_cast<const floatx4*>(arow + k), *reinterpret_cast<const floatx4*>(brow + k));
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][4 * kq + v][i] = acc[v];
    __syncthreads();
  }
  if (!bb_ok) return;

  if (a.dg) {
    const float dhp = red[0][ti][tj] + red[1][ti][tj] + red[2][ti][tj] + red[3][ti][tj] + direct;
    if (!reset_t) dh += dhp;
  }
  const float dn = dh * (1.f - z);
  const float dz = dh * (hp - n);
  const float dan = dn * (1.f - n * n);
  const float dr = dan * hn;
  const float dhn = dan * r;
  const float daz = dz * z * (1.f - z);
  const float dar = dr * r * (1.f - r);
  a.dh_s[(int64_t)bb * a.lddhs + u] = dh;
  float* o = a.dgate_s + (int64_t)bb * a.lddgs;
  o[u] = dan;
  o[H + u] = dar;
  o[2 * H + u] = daz;
  o[3 * H + u] = dhn;
}

// out[s * T * Bm + t * Bm + b] = t * N + envs[s * Bm + b]: the flattened
// sample index of sequence b at step t of env-major minibatch s, listed
// time-major.
__global__ void sequence_rows_kernel(const int32_t* envs, int S, int T, int N, int Bm, int32_t* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per = (int64_t)T * Bm;
  if (i >= (int64_t)S * per) return;
  const int s = (int)(i / per);
  const int64_t r = i - (int64_t)s * per;
  const int t = (int)(r / Bm);
  const int b = (int)(r - (int64_t)t * Bm);
  out[i] = t * N + envs[(int64_t)s * Bm + b];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

PPO_EXPORT int ppo_gru_fwd_step_f32(void* stream, const float* xi, int64_t ldxi, const float* hprev, int64_t ldh,
                                    const int32_t* hprev_rows, const uint8_t* terminated,
                                    const uint8_t* truncated, const int32_t* flag_rows, const float* wh,
                                    int64_t ldwh, const float* bhn, float* h_out, int64_t ldo, float* hp_out,
                                    int64_t ldhp, float* gates, int64_t ldg, int Bm, int H) {
  if (Bm < 0 || H <= 0 || H % 64 != 0)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_step_f32: need Bm >= 0 and H a positive multiple of 64 "
                          "(Bm=%d H=%d)", Bm, H);
  if (Bm == 0) return PPO_OK;
  if (!xi || !hprev || !wh || !bhn || !h_out)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_step_f32: null buffer");
  if (ldxi < 3 * H || ldh < H || ldwh < 3 * H || ldo < H || (hp_out && ldhp < H) || (gates && ldg < 4 * H))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_step_f32: leading dimension too small");
  if (!aligned16(hprev) || ldh % 4 != 0)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_step_f32: hprev rows must be 16-byte aligned");
  FwdArgs a{xi, ldxi, hprev, ldh, hprev_rows, terminated, truncated, flag_rows, wh, ldwh, bhn,
            h_out, ldo, hp_out, ldhp, gates, ldg, Bm, H};
  dim3 grid(ppo::ceil_div(Bm, TILE), H / TILE);
  hipStream_t st = ppo::as_stream(stream);
  switch (H / 64) {  // 16-wide k steps per wave
    case 1: hipLaunchKernelGGL(gru_fwd_step_kernel<1>, grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(gru_fwd_step_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(gru_fwd_step_kernel<4>, grid, dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL(gru_fwd_step_kernel<8>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(gru_fwd_step_kernel<0>, grid, dim3(256), 0, st, a); break;
  }
  return ppo::check_launch("ppo_gru_fwd_step_f32");
}

PPO_EXPORT int ppo_gru_bwd_step_f32(void* stream, const float* dg, int64_t lddg, const float* wh, int64_t ldwh,
                                    const float* dh_t, int64_t lddht, const float* z_t, int64_t ldz,
                                    const uint8_t* terminated, const uint8_t* truncated,
                                    const int32_t* flag_rows, const float* dout, int64_t lddo,
                                    const float* gates_s, int64_t ldg, const float* hp_s, int64_t ldhp,
                                    float* dh_s, int64_t lddhs, float* dgate_s, int64_t lddgs, int Bm, int H) {
  if (Bm < 0 || H <= 0 || H % 64 != 0)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_step_f32: need Bm >= 0 and H a positive multiple of 64 "
                          "(Bm=%d H=%d)", Bm, H);
  if (Bm == 0) return PPO_OK;
  if (!dout || !gates_s || !hp_s || !dh_s || !dgate_s)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_step_f32: null buffer");
  if (dg && (!wh || !dh_t || !z_t))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_step_f32: a step contraction needs wh, dh_t and z_t");
  if (lddo < H || ldg < 4 * H || ldhp < H || lddhs < H || lddgs < 4 * H ||
      (dg && (lddg < 3 * H || ldwh < 3 * H || lddht < H || ldz < H)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_step_f32: leading dimension too small");
  if (dg && (!aligned16(dg) || !aligned16(wh) || lddg % 4 != 0 || ldwh % 4 != 0))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_step_f32: dg and wh rows must be 16-byte aligned");
  BwdArgs a{dg, lddg, wh, ldwh, dh_t, lddht, z_t, ldz, terminated, truncated, flag_rows,
            dout, lddo, gates_s, ldg, hp_s, ldhp, dh_s, lddhs, dgate_s, lddgs, Bm, H};
  dim3 grid(ppo::ceil_div(Bm, TILE), H / TILE);
  hipStream_t st = ppo::as_stream(stream);
  switch (3 * H / 64) {  // 16-wide k steps per wave
    case 3: hipLaunchKernelGGL(gru_bwd_step_kernel<3>, grid, dim3(256), 0, st, a); break;
    case 6: hipLaunchKernelGGL(gru_bwd_step_kernel<6>, grid, dim3(256), 0, st, a); break;
    case 12: hipLaunchKernelGGL(gru_bwd_step_kernel<12>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(gru_bwd_step_kernel<0>, grid, dim3(256), 0, st, a); break;
  }
  return ppo::check_launch("ppo_gru_bwd_step_f32");
}

PPO_EXPORT int ppo_sequence_rows(void* stream, const int32_t* envs, int S, int T, int N, int Bm, int32_t* out) {
  if (S < 0 || T < 0 || N < 0 || Bm < 0 || Bm > N)
    return ppo::set_error(PPO_ERR_ARG, "ppo_sequence_rows: bad shape S=%d T=%d N=%d Bm=%d", S, T, N, Bm);
  if ((int64_t)T * N > INT32_MAX) return ppo::set_error(PPO_ERR_ARG, "ppo_sequence_rows: T * N overflows int32");
  const int64_t n = (int64_t)S * T * Bm;
  if (n == 0) return PPO_OK;
  if (!envs || !out) return ppo::set_error(PPO_ERR_ARG, "ppo_sequence_rows: null buffer");
  hipLaunchKernelGGL(sequence_rows_kernel, dim3((unsigned)ppo::ceil_div64(n, 256)), dim3(256), 0,
                     ppo::as_stream(stream), envs, S, T, N, Bm, out);
  return ppo::check_launch("ppo_sequence_rows");
}
