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

// No multiply-add contraction in this file: the step and sequence kernels
// round every operation alike, whatever their scheduling.
#pragma clang fp contract(off)

namespace {

constexpr int TILE = 16;
constexpr int WAVES = 4;

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }

// The cell arithmetic of one (sequence, unit), forward and backward, with
// every rounding step explicit so that the step and sequence kernels
// (compiled apart) produce the same bits.
__device__ __forceinline__ float gru_cell_fwd(float xr, float ar, float xz, float az, float xn, float an, float bhn,
                                              float hp, float& r, float& z, float& hn, float& n) {
  r = sigmoidf_(xr + ar);
  z = sigmoidf_(xz + az);
  hn = an + bhn;
  n = tanhf(__fmaf_rn(r, hn, xn));                       // xn + r hn
  return __fmaf_rn(z, hp, __fmul_rn(1.f - z, n));        // (1 - z) n + z hp
}
__device__ __forceinline__ void gru_cell_bwd(float dh, float n, float r, float z, float hn, float hp, float& dan,
                                             float& dar, float& daz, float& dhn) {
  const float dn = __fmul_rn(dh, 1.f - z);
  const float dz = __fmul_rn(dh, hp - n);
  dan = __fmul_rn(dn, __fmaf_rn(-n, n, 1.f));            // dn (1 - n^2)
  const float dr = __fmul_rn(dan, hn);
  dhn = __fmul_rn(dan, r);
  daz = __fmul_rn(__fmul_rn(dz, z), 1.f - z);
  dar = __fmul_rn(__fmul_rn(dr, r), 1.f - r);
}

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
  float r, z, hn, n;
  const float h = gru_cell_fwd(xr, ar, xz, az, xn, an, bhn, hp, r, z, hn, n);
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
    direct = __fmul_rn(a.dh_t[(int64_t)bbc * a.lddht + u], a.z_t[(int64_t)bbc * a.ldz + u]);
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
  float dan, dar, daz, dhn;
  gru_cell_bwd(dh, n, r, z, hn, hp, dan, dar, daz, dhn);
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

// ------------------------------------------------- persistent recurrence
// The whole sequence in one launch per direction.  Workgroup (x, y) owns
// sequences 16 x .. 16 x + 15 and units 16 y .. 16 y + 15 for every step; each
// lane holds its slice of the recurrent kernel in registers for the whole
// launch.  Step t of a sequence block needs only the previous step of the
// same block, produced by the gridDim.y workgroups that share x.  They hand it
// over through an exchange ring of two slots, each [Bm][K] 64-bit pairs
// {value bits, tag} (K = H forward, 3H backward), zeroed at launch: a
// producer stores each value with the tag of its step (device-coherent 64-bit
// stores, which land whole), and each consumer wave loads the pairs of its
// own quarter of K for the block's 16 rows (device-coherent 64-bit loads,
// each load of the wave 64 consecutive pairs), reloading those whose tag is
// not yet the step's, and stages them in an LDS tile of its own for the
// contraction.  No counter, no fence: a value is read only once its own tag
// says it is there.  The contraction and epilogue of a step are those of the
// one-step kernels, so the results are the same bits.
//
// Waves of one workgroup meet once per step, where the four partial tiles are
// summed; a wave may run one step ahead of another, so the partial tiles
// alternate between two LDS buffers.  A wave writes a buffer again two steps
// later only after it has read, from some producer, values that producer
// wrote after its own waves had read all 16 rows of this workgroup's previous
// step (each producer's waves together read every column), and this
// workgroup's waves put those rows out only after summing the buffer.  The
// same chain keeps the ring: a slot is written again two steps later only
// after its producer has consumed the step in between, which every consumer
// of the slot produced after reading it.  A wait polls at most spin_limit
// times (0: not at all, which tests the error path from the host): when one
// gives up it sets *error and records its step in LDS, and after that step's
// meeting every wave of the workgroup returns, so every workgroup ends.

typedef unsigned long long u64;

struct SeqSync {
  u64* ring;     // [2][Bm][K] pairs, zero at launch
  int* error;    // set to 1 when a wait gave up
  int spin_limit;
  u64* clear;    // or null: the other direction's ring, which the launch leaves zero
  int64_t clear_n;  // its pairs
};

// This workgroup's share of the other direction's ring, zeroed by its
// recurrence waves (threads 0 .. 255) as they finish, so that the next
// launch, which exchanges through it, needs no zeroing launch before it.
__device__ __forceinline__ void clear_share(const SeqSync& s, int tid) {
  if (!s.clear) return;
  const int64_t nwg = (int64_t)gridDim.x * gridDim.y, wg = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
  const int64_t per = (s.clear_n + nwg - 1) / nwg;
  const int64_t b = wg * per, e = min(s.clear_n, b + per);
  for (int64_t i = b + tid; i < e; i += 256) s.clear[i] = 0ull;
}

__device__ __forceinline__ void put_pair(u64* p, float v, unsigned tag) {
  __hip_atomic_store(p, ((u64)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned tag_of(u64 p) { return (unsigned)(p >> 32); }

// Waits until the wave's quarter of a ring slot's columns, kw .. kw + KW - 1
// of rows b0 .. b0 + 15 ([Bm][K] pairs), carries `tag`, and stages it in the
// wave's own LDS tile sA[16][KW + 4] (rows from Bm on are staged as zeros).
// Each load of the wave reads 64 consecutive pairs of the tile's rows.  Only
// this wave writes and reads sA, and a wave's LDS accesses complete in
// order, so no barrier follows.  Returns false, alike in every lane, when
// spin_limit polls went by without all of them there.
// EAGER: the first round loads every pair unconditionally (rows from Bm on
// read row b0's) before the first check, which the forward's 16 loads per
// lane run faster (212 -> 193 us per 64-step launch at 256 x 256); the
// backward's 48 loads per lane run faster issued inside the polling loop,
// each only while its pair is missing (310 against 414 us).
// signal (may be null): set to sig once the first round of loads is issued
// (a hint for the waves that share this wave's SIMD; see the backward).
template <int K, int KW, bool EAGER>
__device__ __forceinline__ bool stage_wave(const u64* slot, int Bm, int b0, int kw, unsigned tag, float* sA,
                                           int spin_limit, int* signal = nullptr, int sig = 0) {
  auto raise = [&]() {
    if (signal) {
      __builtin_amdgcn_sched_barrier(0);
      __hip_atomic_store(signal, sig, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  constexpr int NL = TILE * KW / 64;
  static_assert(TILE * KW % 64 == 0, "rows of KW pairs over a wave");
  const int lane = threadIdx.x & 63;
  auto at = [&](int q) {
    const int e = lane + 64 * q, r = e / KW;
    return slot + (int64_t)(b0 + r < Bm ? b0 + r : b0) * K + kw + (e - r * KW);
  };
  auto in_rows = [&](int q) { return b0 + (lane + 64 * q) / KW < Bm; };
  u64 v[NL];
  bool ok = false;
  if constexpr (EAGER) {
#pragma unroll
    for (int q = 0; q < NL; ++q) v[q] = __hip_atomic_load(at(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    raise();
    for (int polls = 1;; ++polls) {
      bool mine = true;
#pragma unroll
      for (int q = 0; q < NL; ++q) mine = mine && (!in_rows(q) || tag_of(v[q]) == tag);
      if (spin_limit > 0 && __builtin_amdgcn_ballot_w64(!mine) == 0) {
        ok = true;
        break;
      }
      if (polls >= spin_limit) break;
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int q = 0; q < NL; ++q)
        if (in_rows(q) && tag_of(v[q]) != tag)
          v[q] = __hip_atomic_load(at(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
#pragma unroll
    for (int q = 0; q < NL; ++q) v[q] = in_rows(q) ? 0ull : (u64)tag << 32;
    for (int it = 0; it < spin_limit; ++it) {
      bool mine = true;
#pragma unroll
      for (int q = 0; q < NL; ++q) {
        if (tag_of(v[q]) != tag) {
          const int e = lane + 64 * q, r = e / KW;
          v[q] = __hip_atomic_load(slot + (int64_t)(b0 + r) * K + kw + (e - r * KW), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (it == 0) raise();
#pragma unroll
      for (int q = 0; q < NL; ++q) mine = mine && tag_of(v[q]) == tag;
      if (__builtin_amdgcn_ballot_w64(!mine) == 0) {
        ok = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (spin_limit <= 0) raise();
  }
#pragma unroll
  for (int q = 0; q < NL; ++q) {
    const int e = lane + 64 * q, r = e / KW;
    // (not EAGER: a row from Bm on holds the tag and zero value bits)
    sA[r * (KW + 4) + (e - r * KW)] = !EAGER || in_rows(q) ? __uint_as_float((uint32_t)v[q]) : 0.f;
  }
  __builtin_amdgcn_wave_barrier();
  return ok;
}

// The reset flags of the block's 16 rows for FLAG_CHUNK steps, read once per
// chunk (their row-table lookups are chains of dependent loads, kept off each
// step's path): done[j][r] = whether row b0 + r is done at step step0 + dir j
// (1 for rows from Bm on and steps outside [0, T)).  Barriers on both sides,
// so no thread still reads the previous chunk.
constexpr int FLAG_CHUNK = 64;

__device__ __forceinline__ void load_flag_chunk(uint8_t (*done)[TILE], const uint8_t* term, const uint8_t* trunc,
                                                const int32_t* flag_rows, int64_t flag_step, int Bm, int T, int b0,
                                                int step0, int dir) {
  __syncthreads();
  for (int e = threadIdx.x; e < FLAG_CHUNK * TILE; e += blockDim.x) {
    const int j = e / TILE, r = e - j * TILE;
    const int t = step0 + dir * j, b = b0 + r;
    uint8_t d = 1;
    if (t >= 0 && t < T && b < Bm) d = done_at(term, trunc, flag_rows ? flag_rows + t * flag_step : nullptr, b);
    done[j][r] = d;
  }
  __syncthreads();
}

__global__ void zero_u64_kernel(u64* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0ull;
}

struct FwdSeqArgs {
  const float* xi; int64_t ldxi, xi_step;
  const float* h0; int64_t ldh0; const int32_t* h0_rows;
  const uint8_t* term; const uint8_t* trunc; const int32_t* flag_rows; int64_t flag_step;
  const float* wh; int64_t ldwh;
  const float* bhn;
  float* h_out; int64_t ldo, h_step;
  float* hp_out; int64_t ldhp, hp_step;
  float* gates; int64_t ldg, g_step;
  int Bm, H, T;
  SeqSync sync;
  // XW kernels: the input projections xi = e Wi + bi made in the launch from
  // the GRU input e of row t Bm + b at e + t e_step + b lde (xi unused)
  const float* e; int64_t lde, e_step;
  const float* wi; int64_t ldwi;
  const float* bi;
};

// Input projections inside the forward (XW): four more waves (two per SIMD)
// multiply step t's input rows of the workgroup's 16 sequences with its 48
// columns of Wi ([n|r|z] of its 16 units), each wave a quarter of the 256
// inputs with its slice of Wi in registers, between the waves' meetings of
// steps t - 1 and t; the four partial tiles go to an LDS pair of buffers and
// the recurrence's epilogue of step t adds them in wave order, then the bias.
// Each MFMA group is followed by idle cycles so that the recurrence wave of
// its SIMD keeps issuing (the backward's weight-gradient waves measured the
// same).  Every wave passes every barrier (the flag chunks' too).
template <int NIT, bool XW>
__global__ void __launch_bounds__(XW ? 512 : 256) gru_fwd_seq_kernel(FwdSeqArgs a) {
  constexpr int H = 64 * NIT;
  static_assert(!XW || H == 256, "the input projections in the launch take H = 256 (and a 256-wide input)");
  __shared__ float red[2][WAVES][3][TILE][TILE + 1];
  __shared__ float sA[WAVES][TILE * (H / WAVES + 4)];  // each wave's staged quarter of the previous h
  __shared__ uint8_t done[FLAG_CHUNK][TILE];
  __shared__ float sxi[XW ? 2 : 1][WAVES][3][TILE][TILE + 1];  // XW: [step % 2][wave][n|r|z][row][unit]
  __shared__ int gave_up;  // the step at which a wait gave up, -1 while none has
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int b0 = blockIdx.x * TILE;
  const int u0 = blockIdx.y * TILE;
  const int i = lane & 15;
  const int kq = lane >> 4;
  if constexpr (XW) {
    if (wave >= WAVES) {
      // this lane's inputs k = kx + 16 c + q (c, q < 4) of the wave's quarter
      const int kx = 64 * (wave - WAVES) + 4 * kq;
      float bw[4][3][4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int g = 0; g < 3; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) bw[c][g][q] = a.wi[(int64_t)(kx + 16 * c + q) * a.ldwi + g * H + u0 + i];
      // (a row from Bm on reads row b0: its projections are never used)
      const int row = b0 + i < a.Bm ? b0 + i : b0;
      floatx4 ea[4];
      auto load_e = [&](int t) {
        const float* er = a.e + t * a.e_step + (int64_t)row * a.lde + kx;
#pragma unroll
        for (int c = 0; c < 4; ++c) ea[c] = *reinterpret_cast<const floatx4*>(er + 16 * c);
      };
      load_e(0);
      for (int t = 0; t < a.T; ++t) {
        const int j = t % FLAG_CHUNK;
        if (j == 0) load_flag_chunk(done, a.term, a.trunc, a.flag_rows, a.flag_step, a.Bm, a.T, b0, t, 1);
        floatx4 acc[3];
#pragma unroll
        for (int g = 0; g < 3; ++g) acc[g] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int g = 0; g < 3; ++g)
              acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(ea[c][q], bw[c][g][q], acc[g], 0, 0, 0);
            // (the idle gap)
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
          }
        float (*xt)[3][TILE][TILE + 1] = sxi[t & 1];
#pragma unroll
        for (int g = 0; g < 3; ++g)
#pragma unroll
          for (int v = 0; v < 4; ++v) xt[wave - WAVES][g][4 * kq + v][i] = acc[g][v];
        if (t + 1 < a.T) load_e(t + 1);
        __syncthreads();  // the meeting of step t: its projections are in sxi
        if (gave_up == t) return;
      }
      return;
    }
  }
  // this lane's columns: k0 + 16 c + q, c < NIT, q < 4 (the wave's quarter of H)
  const int k0 = wave * (H / WAVES) + 4 * kq;
  float* sAw = sA[wave];
  float bv[NIT][3][4];
#pragma unroll
  for (int c = 0; c < NIT; ++c)
#pragma unroll
    for (int g = 0; g < 3; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[c][g][q] = a.wh[(int64_t)(k0 + 16 * c + q) * a.ldwh + g * H + u0 + i];

  const int ti = tid >> 4;
  const int tj = tid & 15;
  const int bb = b0 + ti;
  const int u = u0 + tj;
  const bool bb_ok = bb < a.Bm;
  const int bbc = bb_ok ? bb : b0;
  const bool row_in = b0 + i < a.Bm;  // the lane's A row
  const int rowc = row_in ? b0 + i : b0;
  const float bhn = a.bhn[u];
  const int64_t slot_size = (int64_t)a.Bm * H;
  // this thread's input projections, loaded a step ahead (XW: made by the
  // projection waves), and its own previous h (no other workgroup writes them)
  const float* x = XW ? nullptr : a.xi + (int64_t)bbc * a.ldxi;
  float xn = 0.f, xr = 0.f, xz = 0.f, bin = 0.f, bir = 0.f, biz = 0.f;
  if constexpr (XW) {
    bin = a.bi[u];
    bir = a.bi[H + u];
    biz = a.bi[2 * H + u];
  } else {
    xn = x[u];
    xr = x[H + u];
    xz = x[2 * H + u];
  }
  float hp_raw = a.h0[(a.h0_rows ? (int64_t)a.h0_rows[bbc] : (int64_t)bbc) * a.ldh0 + u];
  if (tid == 0) gave_up = -1;  // (published by the first flag chunk's barriers)

  for (int t = 0; t < a.T; ++t) {
    const int j = t % FLAG_CHUNK;
    if (j == 0) load_flag_chunk(done, a.term, a.trunc, a.flag_rows, a.flag_step, a.Bm, a.T, b0, t, 1);
    const bool reset_e = done[j][ti] != 0;
    const bool live = done[j][i] == 0;  // a reset sequence starts from h = 0
    floatx4 acc[3];
#pragma unroll
    for (int g = 0; g < 3; ++g) acc[g] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto mfma_chunk = [&](int c, const float (&av)[4]) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int g = 0; g < 3; ++g)
          acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[q], bv[c][g][q], acc[g], 0, 0, 0);
      }
    };
    float xn_next = 0.f, xr_next = 0.f, xz_next = 0.f;
    auto load_next = [&]() {
      if (!XW && t + 1 < a.T) {
        const float* xt = x + (t + 1) * a.xi_step;
        xn_next = xt[u];
        xr_next = xt[H + u];
        xz_next = xt[2 * H + u];
      }
    };
    bool ok = true;
    if (t == 0) {
      // the carries entering the sequence, gathered through h0_rows
      const float* h0r = a.h0 + (a.h0_rows ? (int64_t)a.h0_rows[rowc] : (int64_t)rowc) * a.ldh0 + k0;
      load_next();
#pragma unroll
      for (int c = 0; c < NIT; ++c) {
        float av[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) av[q] = live ? h0r[16 * c + q] : 0.f;
        mfma_chunk(c, av);
      }
    } else {
      ok = stage_wave<H, H / WAVES, true>(a.sync.ring + ((t - 1) & 1) * slot_size, a.Bm, b0, wave * (H / WAVES),
                                          (unsigned)t, sAw, a.sync.spin_limit);
      load_next();  // (issued after the wait, so that they do not hold it up)
#pragma unroll
      for (int c = 0; c < NIT; ++c) {
        const floatx4 w = *reinterpret_cast<const floatx4*>(&sAw[i * (H / WAVES + 4) + 16 * c + 4 * kq]);
        float av[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) av[q] = live ? w[q] : 0.f;
        mfma_chunk(c, av);
      }
    }
    if (!ok && lane == 0) {
      __hip_atomic_fetch_or(a.sync.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      gave_up = t;
    }
    float (*rt)[3][TILE][TILE + 1] = red[t & 1];
#pragma unroll
    for (int g = 0; g < 3; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) rt[wave][g][4 * kq + v][i] = acc[g][v];
    __syncthreads();
    if (gave_up == t) return;

    if constexpr (XW) {
      const float (*xt)[3][TILE][TILE + 1] = sxi[t & 1];
      xn = (((xt[0][0][ti][tj] + xt[1][0][ti][tj]) + xt[2][0][ti][tj]) + xt[3][0][ti][tj]) + bin;
      xr = (((xt[0][1][ti][tj] + xt[1][1][ti][tj]) + xt[2][1][ti][tj]) + xt[3][1][ti][tj]) + bir;
      xz = (((xt[0][2][ti][tj] + xt[1][2][ti][tj]) + xt[2][2][ti][tj]) + xt[3][2][ti][tj]) + biz;
    }
    if (bb_ok) {
      float ar = 0.f, az = 0.f, an = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        ar += rt[w][0][ti][tj];
        az += rt[w][1][ti][tj];
        an += rt[w][2][ti][tj];
      }
      const float hp = reset_e ? 0.f : hp_raw;
      float r, z, hn, n;
      const float h = gru_cell_fwd(xr, ar, xz, az, xn, an, bhn, hp, r, z, hn, n);
      if (t + 1 < a.T) put_pair(a.sync.ring + (t & 1) * slot_size + (int64_t)bb * H + u, h, (unsigned)(t + 1));
      a.h_out[t * a.h_step + (int64_t)bb * a.ldo + u] = h;
      if (a.hp_out) a.hp_out[t * a.hp_step + (int64_t)bb * a.ldhp + u] = hp;
      if (a.gates) {
        float* g = a.gates + t * a.g_step + (int64_t)bb * a.ldg;
        g[u] = n;
        g[H + u] = r;
        g[2 * H + u] = z;
        g[3 * H + u] = hn;
      }
      hp_raw = h;
    }
    if constexpr (!XW) {
      xn = xn_next;
      xr = xr_next;
      xz = xz_next;
    }
  }
  clear_share(a.sync, threadIdx.x);
}

struct BwdSeqArgs {
  const float* wh; int64_t ldwh;
  const uint8_t* term; const uint8_t* trunc; const int32_t* flag_rows; int64_t flag_step;
  const float* dout; int64_t lddo, dout_step;
  const float* gates; int64_t ldg, g_step;
  const float* hp; int64_t ldhp, hp_step;
  float* dh; int64_t lddh, dh_step;
  float* dgate; int64_t lddg, dg_step;
  int Bm, H, T;
  SeqSync sync;
  // DW kernels: the weight gradients of both GRU kernels, one partial per
  // sequence block x (rows 16 x .. 16 x + 15, every step):
  //   whpart[x][k][c] = sum hp[k] dgate[H + c]   (k < H, c < 3H: [dar|daz|dhn])
  //   wipart[x][k][c] = sum e[k] dgate[c]        (k < H, c < 3H: [dan|dar|daz])
  //   whbpart[x][c], wibpart[x][c]: the column sums of dgate[H + c], dgate[c]
  // where e is the GRU input of row t Bm + b at e + t e_step + b lde.
  const float* e; int64_t lde, e_step;
  float* whpart; float* whbpart; float* wipart; float* wibpart;
};

// Weight gradients inside the backward (DW): the workgroup has four more
// waves (two per SIMD), which multiply while the recurrence's waves wait for
// their exchange loads.  The recurrence's epilogue of step s leaves the
// step's dgate tile (16 rows x the workgroup's 16 units x 4 gates) in an LDS
// pair of buffers; while the recurrence stages step s - 2, the
// weight-gradient waves add the tile's products into their 64 of the K rows
// of both partials: k = 64 w + 16 (lane / 16) + 4 v + mt for accumulator
// [mt][gate] element v (the MFMA's M index read as k = 64 w + 4 m + mt, so
// that a lane's A operand is one 16-byte load of 4 consecutive k), the
// block's rows as the MFMA's K (row 4 (lane / 16) + j at k-step j).  Every
// wave passes every barrier (the flag chunks' too): a buffer is written
// after the meeting of step s, read before the meeting of step s - 2 and
// written again after it.  MFMAs of one wave hold up the VALU work of the
// other wave on its SIMD (measured: the recurrence's epilogue took 4 700
// instead of 1 950 cycles with them beside it), so a weight-gradient wave
// starts its products only once the recurrence wave of its SIMD has issued
// the step's exchange loads (stage flag in LDS; a hint for the schedule
// only, the barriers order the data), and they run under the loads' latency.
template <int NIT, bool DW>
__global__ void __launch_bounds__(DW ? 512 : 256) gru_bwd_seq_kernel(BwdSeqArgs a) {
  constexpr int H3 = 64 * NIT;
  constexpr int H = H3 / 3;
  static_assert(!DW || H == 256, "the fused weight gradients take H = 256 (and a 256-wide input)");
  __shared__ float red[2][WAVES][TILE][TILE + 1];
  __shared__ float sA[WAVES][TILE * (H3 / WAVES + 4)];  // each wave's staged quarter of dgate_{s+1}[:, H:4H]
  __shared__ uint8_t done[FLAG_CHUNK][TILE];
  __shared__ float sdg[DW ? 2 : 1][4][TILE][TILE + 4];   // [step % 2][dan|dar|daz|dhn][unit][row]
  __shared__ int gave_up;  // the step at which a wait gave up, -1 while none has
  __shared__ int staging[WAVES];  // DW: the step whose exchange loads recurrence wave w has issued
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int b0 = blockIdx.x * TILE;
  const int u0 = blockIdx.y * TILE;
  const int i = lane & 15;
  const int kq = lane >> 4;
  if constexpr (DW) {
    if (wave >= WAVES) {
      const int g4 = 4 * kq;                        // this lane's rows g4 + j of the block
      const int kd = 64 * (wave - WAVES) + 4 * i;   // its 4 consecutive k
      floatx4 acc_h[4][3], acc_i[4][3];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 3; ++nt) acc_h[mt][nt] = acc_i[mt][nt] = floatx4{0.f, 0.f, 0.f, 0.f};
      floatx4 ha[4], ea[4];  // step sd's hp and e rows, loaded a step ahead
      auto dw_load = [&](int sd) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = b0 + g4 + j < a.Bm ? b0 + g4 + j : b0;  // (a row from Bm on has a zero dgate)
          ha[j] = *reinterpret_cast<const floatx4*>(a.hp + sd * a.hp_step + (int64_t)row * a.ldhp + kd);
          ea[j] = *reinterpret_cast<const floatx4*>(a.e + sd * a.e_step + (int64_t)row * a.lde + kd);
        }
      };
      auto dw_step = [&](int sd) {
        floatx4 bg[4];
#pragma unroll
        for (int gate = 0; gate < 4; ++gate)
          bg[gate] = *reinterpret_cast<const floatx4*>(&sdg[sd & 1][gate][i][g4]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 3; ++nt) {
              acc_h[mt][nt] =
                  __builtin_amdgcn_mfma_f32_16x16x4f32(ha[j][mt], bg[nt + 1][j], acc_h[mt][nt], 0, 0, 0);
              acc_i[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ea[j][mt], bg[nt][j], acc_i[mt][nt], 0, 0, 0);
            }
      };
      dw_load(a.T - 1);
      for (int s = a.T - 1; s >= 0; --s) {
        const int t = s + 1;
        const int j = (a.T - 1 - s) % FLAG_CHUNK;
        if (j == 0) load_flag_chunk(done, a.term, a.trunc, a.flag_rows, a.flag_step, a.Bm, a.T, b0, t, -1);
        if (t < a.T) {
          if (s + 2 < a.T) {
            // step s + 2's tile (written before the meeting of step s + 1),
            // once the recurrence wave of this SIMD has issued step s's loads
            for (int p = 0; p < (1 << 14) &&
                            __hip_atomic_load(&staging[wave - WAVES], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) > s;
                 ++p)
              __builtin_amdgcn_s_sleep(1);
            dw_step(s + 2);
            dw_load(s + 1);
          }
          __syncthreads();  // the meeting of step s
          if (gave_up == s) return;
        }
      }
      __syncthreads();  // step 0's tile
      if (a.T >= 2) {
        dw_step(1);
        dw_load(0);
      }
      dw_step(0);
      __syncthreads();  // (the recurrence waves' column sums)
      const int64_t xk = (int64_t)blockIdx.x * H;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 3; ++nt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int k = 64 * (wave - WAVES) + 16 * kq + 4 * v + mt;
            const int64_t c = nt * H + u0 + i;
            a.whpart[(xk + k) * 3 * H + c] = acc_h[mt][nt][v];
            a.wipart[(xk + k) * 3 * H + c] = acc_i[mt][nt][v];
          }
      return;
    }
  }
  // this lane's columns: k0 + 16 c + q, c < NIT, q < 4 (the wave's quarter of 3H)
  const int k0 = wave * (H3 / WAVES) + 4 * kq;
  float* sAw = sA[wave];
  float bv[NIT][4];
#pragma unroll
  for (int c = 0; c < NIT; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[c][q] = a.wh[(int64_t)(u0 + i) * a.ldwh + k0 + 16 * c + q];

  const int ti = tid >> 4;
  const int tj = tid & 15;
  const int bb = b0 + ti;
  const int u = u0 + tj;
  const bool bb_ok = bb < a.Bm;
  const int bbc = bb_ok ? bb : b0;
  const bool live = b0 + i < a.Bm;  // the lane's A row
  const int64_t slot_size = (int64_t)a.Bm * H3;
  // step s's own operands, loaded a step ahead (no other workgroup writes
  // them); dh and z of step s + 1 stay in registers from that step
  auto own = [&](int s, float& dout, float& n, float& r, float& z, float& hn, float& hp) {
    dout = a.dout[s * a.dout_step + (int64_t)bbc * a.lddo + u];
    const float* gs = a.gates + s * a.g_step + (int64_t)bbc * a.ldg;
    n = gs[u];
    r = gs[H + u];
    z = gs[2 * H + u];
    hn = gs[3 * H + u];
    hp = a.hp[s * a.hp_step + (int64_t)bbc * a.ldhp + u];
  };
  float dout, n, r, z, hn, hp;
  own(a.T - 1, dout, n, r, z, hn, hp);
  float dh_t = 0.f, z_t = 0.f;
  if (tid == 0) gave_up = -1;  // (published by the first flag chunk's barriers)
  if (DW && tid < WAVES) staging[tid] = a.T;  // (no step issued yet; published likewise)

  float bsum[4] = {0.f, 0.f, 0.f, 0.f};  // DW: this thread's column sums of dan, dar, daz, dhn

  for (int s = a.T - 1; s >= 0; --s) {
    const int t = s + 1;
    float dh = dout;
    float dout_n = 0.f, n_n = 0.f, r_n = 0.f, z_n = 0.f, hn_n = 0.f, hp_n = 0.f;
    const int j = (a.T - 1 - s) % FLAG_CHUNK;   // resets of step t = T - (T - 1 - s)
    if (j == 0) load_flag_chunk(done, a.term, a.trunc, a.flag_rows, a.flag_step, a.Bm, a.T, b0, t, -1);
    if (t < a.T) {
      // this thread's own dh_t and step t's update gate and resets
      const float direct = __fmul_rn(dh_t, z_t);
      const bool reset_t = done[j][ti] != 0;
      // dhp[b][u] = sum_c dgate_t[b][H + c] Wh[u][c], c < 3H
      const bool ok = stage_wave<H3, H3 / WAVES, false>(a.sync.ring + (t & 1) * slot_size, a.Bm, b0,
                                                        wave * (H3 / WAVES), (unsigned)(a.T - t), sAw,
                                                        a.sync.spin_limit, DW ? &staging[wave] : nullptr, s);
      // (issued after the wait, so that they do not hold it up)
      if (s > 0) own(s - 1, dout_n, n_n, r_n, z_n, hn_n, hp_n);
      floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NIT; ++c) {
        const floatx4 w = *reinterpret_cast<const floatx4*>(&sAw[i * (H3 / WAVES + 4) + 16 * c + 4 * kq]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x = live ? w[q] : 0.f;
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x, bv[c][q], acc, 0, 0, 0);
        }
      }
      if (!ok && lane == 0) {
        __hip_atomic_fetch_or(a.sync.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        gave_up = s;
      }
      float (*rs)[TILE][TILE + 1] = red[s & 1];
#pragma unroll
      for (int v = 0; v < 4; ++v) rs[wave][4 * kq + v][i] = acc[v];
      __syncthreads();
      if (gave_up == s) return;
      if (bb_ok) {
        const float dhp = rs[0][ti][tj] + rs[1][ti][tj] + rs[2][ti][tj] + rs[3][ti][tj] + direct;
        if (!reset_t) dh += dhp;
      }
    } else if (s > 0) {
      own(s - 1, dout_n, n_n, r_n, z_n, hn_n, hp_n);
    }
    float dan = 0.f, dar = 0.f, daz = 0.f, dhn = 0.f;
    if (bb_ok) {
      gru_cell_bwd(dh, n, r, z, hn, hp, dan, dar, daz, dhn);
      a.dh[s * a.dh_step + (int64_t)bb * a.lddh + u] = dh;
      if (s > 0) {
        u64* o = a.sync.ring + (s & 1) * slot_size + (int64_t)bb * H3;
        const unsigned tag = (unsigned)(a.T - s);
        put_pair(o + u, dar, tag);
        put_pair(o + H + u, daz, tag);
        put_pair(o + 2 * H + u, dhn, tag);
      }
      float* o = a.dgate + s * a.dg_step + (int64_t)bb * a.lddg;
      o[u] = dan;
      o[H + u] = dar;
      o[2 * H + u] = daz;
      o[3 * H + u] = dhn;
    }
    if constexpr (DW) {
      // (zeros for rows from Bm on)
      sdg[s & 1][0][tj][ti] = dan;
      sdg[s & 1][1][tj][ti] = dar;
      sdg[s & 1][2][tj][ti] = daz;
      sdg[s & 1][3][tj][ti] = dhn;
      bsum[0] += dan;
      bsum[1] += dar;
      bsum[2] += daz;
      bsum[3] += dhn;
    }
    dh_t = dh;
    z_t = z;
    dout = dout_n;
    n = n_n;
    r = r_n;
    z = z_n;
    hn = hn_n;
    hp = hp_n;
  }
  if constexpr (DW) {
    __syncthreads();  // step 0's tile is in sdg for the weight-gradient waves
    // the column sums of the block's rows, added in row order
    float* bs = &red[0][0][0][0];
#pragma unroll
    for (int g = 0; g < 4; ++g) bs[(ti * 4 + g) * TILE + tj] = bsum[g];
    __syncthreads();
    const int64_t x3 = (int64_t)blockIdx.x * 3 * H;
    if (tid < 4 * TILE) {
      const int g = tid / TILE, j = tid % TILE;
      float sum = 0.f;
      for (int row = 0; row < TILE; ++row) sum += bs[(row * 4 + g) * TILE + j];
      const int c = u0 + j;
      if (g < 3) a.wibpart[x3 + g * H + c] = sum;          // [dan|dar|daz]
      if (g > 0) a.whbpart[x3 + (g - 1) * H + c] = sum;    // [dar|daz|dhn]
    }
  }
  clear_share(a.sync, tid);
}

int cu_count() {
  static int counts[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    counts[dev] = n;
  }
  return counts[dev];
}

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

// Workgroups a sequence launch runs at once (one per compute unit): the
// sequence entry points need ceil(Bm / 16) * (H / 16) of them at most.
PPO_EXPORT int ppo_gru_seq_max_workgroups() { return cu_count(); }

// Bytes of the exchange ring a sequence launch of either direction needs
// (two slots of [Bm][3H] 64-bit pairs; the launch zeroes what it uses).
PPO_EXPORT int64_t ppo_gru_seq_exchange_bytes(int Bm, int H) {
  return Bm > 0 && H > 0 ? 2 * (int64_t)Bm * 3 * H * (int64_t)sizeof(u64) : 0;
}

// Launches a persistent kernel (one workgroup of 256 threads, 512 with the
// weight-gradient waves, per 16 x 16 tile, all resident at once).
template <typename Kernel, typename Args>
static void launch_seq(Kernel k, dim3 grid, hipStream_t st, const Args& a, int threads = 256) {
  hipLaunchKernelGGL(k, grid, dim3(threads), 0, st, a);
}

static void zero_ring(hipStream_t st, void* ring, int64_t n) {
  const int blocks = (int)std::min<int64_t>(1024, ppo::ceil_div64(n, 256));
  hipLaunchKernelGGL(zero_u64_kernel, dim3(blocks), dim3(256), 0, st, static_cast<u64*>(ring), n);
}

static int seq_check(const char* name, int Bm, int H, int T, const void* exchange, const int* error) {
  if (Bm < 0 || T < 0 || H <= 0 || H % 64 != 0 || H > 256)
    return ppo::set_error(PPO_ERR_ARG, "%s: need Bm, T >= 0 and H in {64, 128, 192, 256} (Bm=%d H=%d T=%d)", name, Bm,
                          H, T);
  if (!exchange || !error) return ppo::set_error(PPO_ERR_ARG, "%s: null exchange ring or error word", name);
  if (!aligned16(exchange)) return ppo::set_error(PPO_ERR_ARG, "%s: exchange ring must be 16-byte aligned", name);
  const int64_t wgs = (int64_t)ppo::ceil_div(Bm, TILE) * (H / TILE);
  const int cus = cu_count();
  if (wgs > cus)
    return ppo::set_error(PPO_ERR_ARG, "%s: %lld workgroups exceed the %d compute units that keep them all resident",
                          name, (long long)wgs, cus);
  return PPO_OK;
}

// Forward of the recurrence over T steps in one launch (see the persistent
// recurrence notes above): step t reads xi + t xi_step and the resets at
// flag_rows + t flag_step, the carry entering step 0 from h0 (rows h0_rows),
// and writes h_out, hp_out and gates at + t times their steps, the values of
// T ppo_gru_fwd_step_f32 launches.  exchange: ppo_gru_seq_exchange_bytes(Bm,
// H) bytes; error: set to 1 if a wait gave up after spin_limit polls.
PPO_EXPORT int ppo_gru_fwd_seq_f32(void* stream, const float* xi, int64_t ldxi, int64_t xi_step, const float* h0,
                                   int64_t ldh0, const int32_t* h0_rows, const uint8_t* terminated,
                                   const uint8_t* truncated, const int32_t* flag_rows, int64_t flag_step,
                                   const float* wh, int64_t ldwh, const float* bhn, float* h_out, int64_t ldo,
                                   int64_t h_step, float* hp_out, int64_t ldhp, int64_t hp_step, float* gates,
                                   int64_t ldg, int64_t g_step, int Bm, int H, int T, void* exchange, int* error,
                                   int spin_limit) {
  const int rc = seq_check("ppo_gru_fwd_seq_f32", Bm, H, T, exchange, error);
  if (rc != PPO_OK) return rc;
  if (Bm == 0 || T == 0) return PPO_OK;
  if (!xi || !h0 || !wh || !bhn || !h_out)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_seq_f32: null buffer");
  if (ldxi < 3 * H || ldh0 < H || ldwh < 3 * H || ldo < H || (hp_out && ldhp < H) || (gates && ldg < 4 * H))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_seq_f32: leading dimension too small");
  if (!aligned16(h0) || ldh0 % 4 || !aligned16(h_out) || ldo % 4 || h_step % 4)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_seq_f32: h0 and h_out rows must be 16-byte aligned");
  FwdSeqArgs a{xi, ldxi, xi_step, h0, ldh0, h0_rows, terminated, truncated, flag_rows, flag_step, wh, ldwh, bhn,
               h_out, ldo, h_step, hp_out, ldhp, hp_step, gates, ldg, g_step, Bm, H, T,
               SeqSync{static_cast<u64*>(exchange), error, spin_limit}, nullptr, 0, 0, nullptr, 0, nullptr};
  hipStream_t st = ppo::as_stream(stream);
  if (T > 1) zero_ring(st, exchange, 2 * (int64_t)Bm * H);
  const dim3 grid(ppo::ceil_div(Bm, TILE), H / TILE);
  switch (H / 64) {
    case 1: launch_seq(gru_fwd_seq_kernel<1, false>, grid, st, a); break;
    case 2: launch_seq(gru_fwd_seq_kernel<2, false>, grid, st, a); break;
    case 3: launch_seq(gru_fwd_seq_kernel<3, false>, grid, st, a); break;
    default: launch_seq(gru_fwd_seq_kernel<4, false>, grid, st, a); break;
  }
  return ppo::check_launch("ppo_gru_fwd_seq_f32");
}

// ppo_gru_fwd_seq_f32 with the input projections made in the launch: xi =
// e Wi + bi for the GRU input e of row t Bm + b at e + t e_step + b lde
// (wi [I][3H] with row pitch ldwi, bi [3H], columns [n|r|z]: the flax
// GRUCell's input Dense kernels, boonta/networks/blocks/rnn.py:34-54),
// each step's products summed in a fixed order (not the order of a separate
// GEMM launch: equal to it to rounding).  H = I = 256; e rows 16-byte aligned.
// ring_is_zero: the exchange ring is already zero (no zeroing launch first);
// clear_ring (clear_bytes, or null / 0): a ring the launch zeroes as its
// workgroups finish — the backward's, so that it needs no zeroing launch
// either (a launch that sets the error word may leave it unzeroed).
PPO_EXPORT int ppo_gru_fwd_seq_xw_f32(void* stream, const float* h0, int64_t ldh0, const int32_t* h0_rows,
                                      const uint8_t* terminated, const uint8_t* truncated, const int32_t* flag_rows,
                                      int64_t flag_step, const float* wh, int64_t ldwh, const float* bhn,
                                      float* h_out, int64_t ldo, int64_t h_step, float* hp_out, int64_t ldhp,
                                      int64_t hp_step, float* gates, int64_t ldg, int64_t g_step, int Bm, int H, int T,
                                      void* exchange, int* error, int spin_limit, const float* e, int64_t lde,
                                      int64_t e_step, int I, const float* wi, int64_t ldwi, const float* bi,
                                      int ring_is_zero, void* clear_ring, int64_t clear_bytes) {
  const int rc = seq_check("ppo_gru_fwd_seq_xw_f32", Bm, H, T, exchange, error);
  if (rc != PPO_OK) return rc;
  if (clear_bytes < 0 || clear_bytes % 8 || (clear_bytes > 0 && (!clear_ring || !aligned16(clear_ring))))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_seq_xw_f32: bad ring to clear (%lld bytes)", (long long)clear_bytes);
  if (H != 256 || I != 256)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_seq_xw_f32: needs H = I = 256 (H=%d I=%d)", H, I);
  if (Bm == 0 || T == 0) return PPO_OK;
  if (!h0 || !wh || !bhn || !h_out || !e || !wi || !bi)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_seq_xw_f32: null buffer");
  if (ldh0 < H || ldwh < 3 * H || ldo < H || (hp_out && ldhp < H) || (gates && ldg < 4 * H) || lde < I ||
      ldwi < 3 * H)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_seq_xw_f32: leading dimension too small");
  if (!aligned16(h0) || ldh0 % 4 || !aligned16(h_out) || ldo % 4 || h_step % 4 || !aligned16(e) || lde % 4 ||
      e_step % 4)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_fwd_seq_xw_f32: h0, h_out and e rows must be 16-byte aligned");
  FwdSeqArgs a{nullptr, 0, 0, h0, ldh0, h0_rows, terminated, truncated, flag_rows, flag_step, wh, ldwh, bhn,
               h_out, ldo, h_step, hp_out, ldhp, hp_step, gates, ldg, g_step, Bm, H, T,
               SeqSync{static_cast<u64*>(exchange), error, spin_limit,
                       clear_bytes > 0 ? static_cast<u64*>(clear_ring) : nullptr, clear_bytes / 8},
               e, lde, e_step, wi, ldwi, bi};
  hipStream_t st = ppo::as_stream(stream);
  if (T > 1 && !ring_is_zero) zero_ring(st, exchange, 2 * (int64_t)Bm * H);
  launch_seq(gru_fwd_seq_kernel<4, true>, dim3(ppo::ceil_div(Bm, TILE), H / TILE), st, a, 512);
  return ppo::check_launch("ppo_gru_fwd_seq_xw_f32");
}

// Backward through time over T steps in one launch: step s (T - 1 down to 0)
// takes the head cotangent dout + s dout_step, gates and hp of step s, and
// for s < T - 1 the contraction of dgate_{s+1}[:, H:4H] with Wh^T, dh_{s+1},
// the update gate and the resets of step s + 1; it writes dh and dgate at
// + s times their steps, the values of T ppo_gru_bwd_step_f32 launches.
PPO_EXPORT int ppo_gru_bwd_seq_f32(void* stream, const float* wh, int64_t ldwh, const uint8_t* terminated,
                                   const uint8_t* truncated, const int32_t* flag_rows, int64_t flag_step,
                                   const float* dout, int64_t lddo, int64_t dout_step, const float* gates,
                                   int64_t ldg, int64_t g_step, const float* hp, int64_t ldhp, int64_t hp_step,
                                   float* dh, int64_t lddh, int64_t dh_step, float* dgate, int64_t lddg,
                                   int64_t dg_step, int Bm, int H, int T, void* exchange, int* error,
                                   int spin_limit) {
  const int rc = seq_check("ppo_gru_bwd_seq_f32", Bm, H, T, exchange, error);
  if (rc != PPO_OK) return rc;
  if (Bm == 0 || T == 0) return PPO_OK;
  if (!wh || !dout || !gates || !hp || !dh || !dgate)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_seq_f32: null buffer");
  if (ldwh < 3 * H || lddo < H || ldg < 4 * H || ldhp < H || lddh < H || lddg < 4 * H)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_seq_f32: leading dimension too small");
  if (!aligned16(dgate) || lddg % 4 || dg_step % 4)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_seq_f32: dgate rows must be 16-byte aligned");
  BwdSeqArgs a{wh, ldwh, terminated, truncated, flag_rows, flag_step, dout, lddo, dout_step, gates, ldg, g_step,
               hp, ldhp, hp_step, dh, lddh, dh_step, dgate, lddg, dg_step, Bm, H, T,
               SeqSync{static_cast<u64*>(exchange), error, spin_limit}, nullptr, 0, 0, nullptr, nullptr, nullptr,
               nullptr};
  hipStream_t st = ppo::as_stream(stream);
  if (T > 1) zero_ring(st, exchange, 2 * (int64_t)Bm * 3 * H);
  const dim3 grid(ppo::ceil_div(Bm, TILE), H / TILE);
  switch (3 * H / 64) {
    case 3: launch_seq(gru_bwd_seq_kernel<3, false>, grid, st, a); break;
    case 6: launch_seq(gru_bwd_seq_kernel<6, false>, grid, st, a); break;
    case 9: launch_seq(gru_bwd_seq_kernel<9, false>, grid, st, a); break;
    default: launch_seq(gru_bwd_seq_kernel<12, false>, grid, st, a); break;
  }
  return ppo::check_launch("ppo_gru_bwd_seq_f32");
}

// Parts of the fused weight gradients of ppo_gru_bwd_seq_dw_f32: one per
// block of 16 sequences.
PPO_EXPORT int ppo_gru_seq_dw_parts(int Bm) { return Bm > 0 ? ppo::ceil_div(Bm, TILE) : 0; }

// ppo_gru_bwd_seq_f32 that also leaves the weight gradients of both GRU
// kernels and their biases as P = ppo_gru_seq_dw_parts(Bm) partials, each
// over the rows of one block of 16 sequences and every step:
//   whpart [P][H][3H]: hp^T dgate[:, H:4H]     whbpart [P][3H]: its column sums
//   wipart [P][I][3H]: e^T dgate[:, 0:3H]      wibpart [P][3H]: its column sums
// with e the GRU input of row t Bm + b at e + t e_step + b lde (the flax
// GRUCell's input and recurrent Dense kernels, boonta/networks/blocks/rnn.py:
// 34-54, differentiated by jax.value_and_grad at
// boonta/algorithms/recurrent_ppo.py:213-215).  H = I = 256; hp and e rows
// 16-byte aligned.  ring_is_zero, clear_ring, clear_bytes: as for
// ppo_gru_fwd_seq_xw_f32 (here clear_ring is the forward's ring).
PPO_EXPORT int ppo_gru_bwd_seq_dw_f32(void* stream, const float* wh, int64_t ldwh, const uint8_t* terminated,
                                      const uint8_t* truncated, const int32_t* flag_rows, int64_t flag_step,
                                      const float* dout, int64_t lddo, int64_t dout_step, const float* gates,
                                      int64_t ldg, int64_t g_step, const float* hp, int64_t ldhp, int64_t hp_step,
                                      float* dh, int64_t lddh, int64_t dh_step, float* dgate, int64_t lddg,
                                      int64_t dg_step, int Bm, int H, int T, void* exchange, int* error,
                                      int spin_limit, const float* e, int64_t lde, int64_t e_step, int I,
                                      float* whpart, float* whbpart, float* wipart, float* wibpart,
                                      int ring_is_zero, void* clear_ring, int64_t clear_bytes) {
  const int rc = seq_check("ppo_gru_bwd_seq_dw_f32", Bm, H, T, exchange, error);
  if (rc != PPO_OK) return rc;
  if (clear_bytes < 0 || clear_bytes % 8 || (clear_bytes > 0 && (!clear_ring || !aligned16(clear_ring))))
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_seq_dw_f32: bad ring to clear (%lld bytes)", (long long)clear_bytes);
  if (H != 256 || I != 256)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_seq_dw_f32: needs H = I = 256 (H=%d I=%d)", H, I);
  if (Bm == 0 || T == 0) return PPO_OK;
  if (!wh || !dout || !gates || !hp || !dh || !dgate || !e || !whpart || !whbpart || !wipart || !wibpart)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_seq_dw_f32: null buffer");
  if (ldwh < 3 * H || lddo < H || ldg < 4 * H || ldhp < H || lddh < H || lddg < 4 * H || lde < I)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_seq_dw_f32: leading dimension too small");
  if (!aligned16(dgate) || lddg % 4 || dg_step % 4 || !aligned16(hp) || ldhp % 4 || hp_step % 4 ||
      !aligned16(e) || lde % 4 || e_step % 4)
    return ppo::set_error(PPO_ERR_ARG, "ppo_gru_bwd_seq_dw_f32: dgate, hp and e rows must be 16-byte aligned");
  BwdSeqArgs a{wh, ldwh, terminated, truncated, flag_rows, flag_step, dout, lddo, dout_step, gates, ldg, g_step,
               hp, ldhp, hp_step, dh, lddh, dh_step, dgate, lddg, dg_step, Bm, H, T,
               SeqSync{static_cast<u64*>(exchange), error, spin_limit,
                       clear_bytes > 0 ? static_cast<u64*>(clear_ring) : nullptr, clear_bytes / 8},
               e, lde, e_step, whpart, whbpart, wipart, wibpart};
  hipStream_t st = ppo::as_stream(stream);
  if (T > 1 && !ring_is_zero) zero_ring(st, exchange, 2 * (int64_t)Bm * 3 * H);
  launch_seq(gru_bwd_seq_kernel<12, true>, dim3(ppo::ceil_div(Bm, TILE), H / TILE), st, a, 512);
  return ppo::check_launch("ppo_gru_bwd_seq_dw_f32");
}
