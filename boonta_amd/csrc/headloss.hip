// Fused policy/value heads + PPO loss + head backward, one pass over the torso
// output of a minibatch.
//
// Follows loss_fn of boonta/algorithms/ppo.py:77-146 (recurrent_ppo.py:101-184)
// with the heads of boonta/networks/heads.py:9-45 (a Dense layer each, or one
// Dense feeding both when actor and critic share the torso) and the
// distributions of boonta/networks/distributions.py:8-57.
//
// Work split: each wavefront owns a run of <= 64 consecutive rows; lane l
// holds features f = l + 64 e (e < VPL) and the matching head-weight rows in
// registers for the whole block.
//   A. one row at a time: the NA head outputs are VPL * NA FMAs per lane and a
//      butterfly reduce-scatter (NA/2 + NA/4 + ... exchanges instead of NA
//      full wave reductions); they go to LDS;
//   B. one lane per row: the loss, its statistics and the cotangents of the
//      head outputs, computed once per row instead of redundantly per lane;
//   C. one row at a time again: the cotangent of the torso output,
//      sum_j dout_j W[f][j] times the derivative of the torso's last
//      activation, is written, and H[f] * dout_j accumulates the head weight
//      gradient in registers.
// Rows are prefetched two ahead in A and C.
// Per-block partials (head weights and biases, Gaussian scale, statistics)
// are folded across the block's waves in a fixed order; the gradient reduce
// kernel sums the blocks.
#include "common.h"

#include <algorithm>

namespace {

constexpr int HL_THREADS = 256;
constexpr int HL_WAVES = HL_THREADS / 64;

enum Dist { DIST_CATEGORICAL = 0, DIST_GAUSSIAN = 1 };
enum Stat {
  ST_ACTOR = 0, ST_ENTROPY, ST_KL, ST_CLIPFRAC, ST_ADV, ST_CRITIC, ST_RESID, ST_RESID2, ST_RET, ST_RET2,
  ST_VALUE, NSTAT
};

struct HeadLossParams {
  int dist, rows;
  const int32_t* idx;
  // group a: the actor head (or both heads, value in the last column, when hc is null)
  const float* ha; int64_t ldha; const float* wa; int64_t ldwa; const float* ba; int na;
  // group c: the critic head (separate towers)
  const float* hc; int64_t ldhc; const float* wc; int64_t ldwc; const float* bc;
  int F;  // feature width of both head inputs
  int A;  // categories, or Gaussian dimension D
  const float* scale_param;  // state-independent raw Gaussian scale [D] or null
  const int32_t* action_i; const float* action_f;
  const float* old_logp; const float* old_value; const float* adv; const float* ret;
  int act_a; const float* aux_a; int64_t ldaux_a; float* dha; int64_t lddha;
  int act_c; const float* aux_c; int64_t ldaux_c; float* dhc; int64_t lddhc;
  float* wpart_a; float* bpart_a; float* wpart_c; float* bpart_c;
  float* dscale_partial; double* stats_partial;
  float clip_eps; int clip_value_loss; float ent_coef, vf_coef, inv_n, temperature;
};

template <int NA>
__device__ __forceinline__ float reduce_scatter(float (&v)[NA], int lane) {
  float buf[NA];
#pragma unroll
  for (int k = 0; k < NA; ++k) buf[k] = v[k];
  int off = 32;
#pragma unroll
  for (int size = NA; size > 1; size >>= 1) {
    const int half = size >> 1;
    const bool hi = (lane & off) != 0;
#pragma unroll
    for (int k = 0; k < half; ++k) {
      const float send = hi ? buf[k] : buf[k + half];
      const float recv = __shfl_xor(send, off, 64);
      buf[k] = (hi ? buf[k + half] : buf[k]) + recv;
    }
    off >>= 1;
  }
#pragma unroll
  for (; off >= 1; off >>= 1) buf[0] += __shfl_xor(buf[0], off, 64);
  return buf[0];
}

template <int NA>
constexpr int log2_of() {
  return NA <= 1 ? 0 : 1 + log2_of<NA / 2>();
}

__device__ __forceinline__ float tie_first(float x, float y, float ans) {
  return (x == ans ? 1.f : 0.f) / (y == ans ? 2.f : 1.f);
}
__device__ __forceinline__ void clip_grad(float x, float lo, float hi, float& out, float& dx) {
  const float m = fmaxf(lo, x);
  const float dm = tie_first(x, lo, m);
  out = fminf(hi, m);
  dx = tie_first(m, hi, out) * dm;
}
__device__ __forceinline__ float softplusf(float x) { return fmaxf(x, 0.f) + log1pf(__expf(-fabsf(x))); }

constexpr float LOG_2PI = 1.8378770664093453f;

template <int VPL, int NA, bool SEP>
__global__ void __launch_bounds__(HL_THREADS) head_loss_kernel(HeadLossParams p) {
  extern __shared__ float smem[];  // fold buffer [F][NA + 1]
  constexpr int NO = NA + 1;       // head outputs + the critic's value (separate towers)
  __shared__ float s_out[HL_WAVES][64][NO];
  __shared__ float s_dout[HL_WAVES][64][NO];
  __shared__ double s_stats[HL_WAVES][NSTAT];
  __shared__ float s_vec[HL_WAVES][3][NA];  // db_a, db_c (col 0), dscale

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  constexpr int P = log2_of<NA>();
  const int F = p.F;
  const int A = p.A;

  // Each wave owns a contiguous run of at most 64 rows (the launch sizes the
  // grid for it): lane k of the wave is the run's k-th row in phase B.
  const int total_waves = gridDim.x * HL_WAVES;
  const int per_wave = (p.rows + total_waves - 1) / total_waves;
  const int gw = blockIdx.x * HL_WAVES + wave;
  const int r_begin = __builtin_amdgcn_readfirstlane(min(p.rows, gw * per_wave));
  const int r_end = __builtin_amdgcn_readfirstlane(min(p.rows, r_begin + per_wave));
  const int R = r_end - r_begin;

  // head weights of this lane's features, in registers for phases A and C
  float wa[VPL][NA];
  float wc[VPL];
#pragma unroll
  for (int e = 0; e < VPL; ++e) {
    const int f = lane + 64 * e;
#pragma unroll
    for (int j = 0; j < NA; ++j) wa[e][j] = (f < F && j < p.na) ? p.wa[(int64_t)f * p.ldwa + j] : 0.f;
    wc[e] = (SEP && f < F) ? p.wc[(int64_t)f * p.ldwc] : 0.f;
  }

  // ---------------- phase A: head outputs of every row, one wavefront per row
  {
    float hb[2][VPL], hcb[2][VPL];
    auto fetch = [&](int row, float (&h)[VPL], float (&hc)[VPL]) {
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        const int f = lane + 64 * e;
        const bool ok = row < r_end && f < F;
        h[e] = ok ? p.ha[(int64_t)row * p.ldha + f] : 0.f;
        hc[e] = (SEP && ok) ? p.hc[(int64_t)row * p.ldhc + f] : 0.f;
      }
    };
    auto step = [&](int k, float (&h)[VPL], float (&hc)[VPL]) {
      float part[NA];
#pragma unroll
      for (int j = 0; j < NA; ++j) part[j] = 0.f;
      float pc = 0.f;
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
#pragma unroll
        for (int j = 0; j < NA; ++j) part[j] += h[e] * wa[e][j];
        pc += hc[e] * wc[e];
      }
      fetch(r_begin + k + 2, h, hc);
      const float mine = reduce_scatter<NA>(part, lane);
      if ((lane & ((64 >> P) - 1)) == 0) s_out[wave][k][lane >> (6 - P)] = mine;
      if (SEP) {
        const float v = ppo::wave_sum(pc);
        if (lane == 0) s_out[wave][k][NA] = v;
      }
    };
    fetch(r_begin, hb[0], hcb[0]);
    fetch(r_begin + 1, hb[1], hcb[1]);
    for (int k = 0; k < R; k += 2) {
      step(k, hb[0], hcb[0]);
      if (k + 1 < R) step(k + 1, hb[1], hcb[1]);
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---------------- phase B: loss and output cotangents, one lane per row
  double st[NSTAT];
#pragma unroll
  for (int i = 0; i < NSTAT; ++i) st[i] = 0.0;
  float db_a[NA], dsc[NA];
#pragma unroll
  for (int j = 0; j < NA; ++j) db_a[j] = dsc[j] = 0.f;
  float db_c = 0.f;
  if (lane < R) {
    const int r = r_begin + lane;
    const int64_t s = p.idx ? (int64_t)p.idx[r] : (int64_t)r;
    const float olp = p.old_logp[s], Av = p.adv[s], Rt = p.ret[s], vold = p.old_value[s];
    const float eps = p.clip_eps;
    const float inv_t = 1.f / p.temperature;
    float out[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) out[j] = s_out[wave][lane][j] + (j < p.na ? p.ba[j] : 0.f);
    const float v = SEP ? s_out[wave][lane][NA] + p.bc[0] : out[p.na - 1];

    float lp = 0.f, ent = 0.f;
    float dout[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) dout[j] = 0.f;
    float lse = 0.f;
    int a = 0;
    if (p.dist == DIST_CATEGORICAL) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < NA; ++j) if (j < A) mx = fmaxf(mx, out[j] * inv_t);
      float se = 0.f;
#pragma unroll
      for (int j = 0; j < NA; ++j) if (j < A) se += __expf(out[j] * inv_t - mx);
      lse = mx + __logf(se);
      a = p.action_i[s];
      float za = -INFINITY;
#pragma unroll
      for (int j = 0; j < NA; ++j) za = (j == a) ? out[j] * inv_t : za;
      lp = (a >= 0 && a < A) ? za - lse : -INFINITY;
#pragma unroll
      for (int j = 0; j < NA; ++j)
        if (j < A) {
          const float lq = out[j] * inv_t - lse;
          ent -= __expf(lq) * lq;
        }
    } else {
#pragma unroll
      for (int j = 0; j < NA; ++j)
        if (j < A) {
          float raw = 0.f;
          if (p.scale_param) {
            raw = p.scale_param[j];
          } else {
#pragma unroll
            for (int q = 0; q < NA; ++q) raw = (q == A + j) ? out[q] : raw;
          }
          const float sig = p.temperature * (softplusf(raw) + 1e-3f);
          const float zz = (p.action_f[s * A + j] - out[j]) / sig;
          const float ls = __logf(sig);
          lp += -0.5f * zz * zz - ls - 0.5f * LOG_2PI;
          ent += 0.5f + 0.5f * LOG_2PI + ls;
        }
    }

    // loss terms and cotangents (jax tie rules for min / max / clip)
    const float ratio = __expf(lp - olp);
    float cr, dcr;
    clip_grad(ratio, 1.f - eps, 1.f + eps, cr, dcr);
    const float pg1 = ratio * Av, pg2 = cr * Av;
    const float pmin = fminf(pg1, pg2);
    const float g_lp = -(tie_first(pg1, pg2, pmin) * Av + tie_first(pg2, pg1, pmin) * Av * dcr) * p.inv_n * ratio;
    const float g_ent = -p.ent_coef * p.inv_n;
    const float vl1 = 0.5f * (v - Rt) * (v - Rt);
    float crow, gv;
    if (p.clip_value_loss) {
      float dv, ddv;
      clip_grad(v - vold, -eps, eps, dv, ddv);
      const float vc = vold + dv;
      const float vl2 = 0.5f * (vc - Rt) * (vc - Rt);
      crow = fmaxf(vl1, vl2);
      gv = tie_first(vl1, vl2, crow) * (v - Rt) + tie_first(vl2, vl1, crow) * (vc - Rt) * ddv;
    } else {
      crow = vl1;
      gv = v - Rt;
    }
    const float dvalue = p.vf_coef * gv * p.inv_n;

    if (p.dist == DIST_CATEGORICAL) {
#pragma unroll
      for (int j = 0; j < NA; ++j)
        if (j < A) {
          const float lq = out[j] * inv_t - lse;
          const float q = __expf(lq);
          dout[j] = (g_lp * ((j == a ? 1.f : 0.f) - q) - g_ent * q * (lq + ent)) * inv_t;
        }
    } else {
#pragma unroll
      for (int j = 0; j < NA; ++j)
        if (j < A) {
          float raw = 0.f;
          if (p.scale_param) {
            raw = p.scale_param[j];
          } else {
#pragma unroll
            for (int q = 0; q < NA; ++q) raw = (q == A + j) ? out[q] : raw;
          }
          const float sig = p.temperature * (softplusf(raw) + 1e-3f);
          const float d = p.action_f[s * A + j] - out[j];
          dout[j] = g_lp * d / (sig * sig);
          const float dsig = g_lp * (d * d / (sig * sig * sig) - 1.f / sig) + g_ent / sig;
          const float draw = dsig * p.temperature / (1.f + __expf(-raw));
          if (p.scale_param) {
            dsc[j] += draw;
          } else {
#pragma unroll
            for (int q = 0; q < NA; ++q) dout[q] = (q == A + j) ? draw : dout[q];
          }
        }
    }
    if (!SEP) {
#pragma unroll
      for (int j = 0; j < NA; ++j) dout[j] = (j == p.na - 1) ? dvalue : dout[j];
    }
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      s_dout[wave][lane][j] = dout[j];
      db_a[j] += dout[j];
    }
    s_dout[wave][lane][NA] = dvalue;
    db_c += dvalue;

    st[ST_ACTOR] += (double)(-pmin);
    st[ST_ENTROPY] += (double)ent;
    st[ST_KL] += (double)(olp - lp);
    st[ST_CLIPFRAC] += (fabsf(ratio - 1.f) > eps) ? 1.0 : 0.0;
    st[ST_ADV] += (double)Av;
    st[ST_CRITIC] += (double)crow;
    const double res = (double)Rt - (double)v;
    st[ST_RESID] += res;
    st[ST_RESID2] += res * res;
    st[ST_RET] += (double)Rt;
    st[ST_RET2] += (double)Rt * (double)Rt;
    st[ST_VALUE] += (double)v;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---------------- phase C: head backward, one wavefront per row
  // The activation derivative reads the layer output itself for relu / tanh
  // (aux == h) and the pre-activation for silu.
  const bool load_xa = p.act_a != ACT_NONE && !(p.aux_a == p.ha && p.ldaux_a == p.ldha);
  const bool load_xc = SEP && p.act_c != ACT_NONE && !(p.aux_c == p.hc && p.ldaux_c == p.ldhc);
  float acc_a[VPL][NA];
  float acc_c[VPL];
#pragma unroll
  for (int e = 0; e < VPL; ++e) {
    acc_c[e] = 0.f;
#pragma unroll
    for (int j = 0; j < NA; ++j) acc_a[e][j] = 0.f;
  }
  {
    float hb[2][VPL], hcb[2][VPL], xab[2][VPL], xcb[2][VPL];
    auto fetch = [&](int row, float (&h)[VPL], float (&hc)[VPL], float (&xa)[VPL], float (&xc)[VPL]) {
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        const int f = lane + 64 * e;
        const bool ok = row < r_end && f < F;
        h[e] = ok ? p.ha[(int64_t)row * p.ldha + f] : 0.f;
        xa[e] = (ok && load_xa) ? p.aux_a[(int64_t)row * p.ldaux_a + f] : h[e];
        hc[e] = (SEP && ok) ? p.hc[(int64_t)row * p.ldhc + f] : 0.f;
        xc[e] = (ok && load_xc) ? p.aux_c[(int64_t)row * p.ldaux_c + f] : hc[e];
      }
    };
    auto step = [&](int k, float (&h)[VPL], float (&hc)[VPL], float (&xa)[VPL], float (&xc)[VPL]) {
      const int r = r_begin + k;
      float dout[NA];
#pragma unroll
      for (int j = 0; j < NA; ++j) dout[j] = s_dout[wave][k][j];
      const float dvalue = s_dout[wave][k][NA];
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        const int f = lane + 64 * e;
        float g = 0.f;
#pragma unroll
        for (int j = 0; j < NA; ++j) {
          g += dout[j] * wa[e][j];
          acc_a[e][j] += h[e] * dout[j];
        }
        if (f < F) {
          if (p.act_a != ACT_NONE) g *= ppo::act_grad(p.act_a, xa[e]);
          p.dha[(int64_t)r * p.lddha + f] = g;
        }
        if (SEP) {
          float gc = dvalue * wc[e];
          acc_c[e] += hc[e] * dvalue;
          if (f < F) {
            if (p.act_c != ACT_NONE) gc *= ppo::act_grad(p.act_c, xc[e]);
            p.dhc[(int64_t)r * p.lddhc + f] = gc;
          }
        }
      }
      fetch(r + 2, h, hc, xa, xc);
    };
    fetch(r_begin, hb[0], hcb[0], xab[0], xcb[0]);
    fetch(r_begin + 1, hb[1], hcb[1], xab[1], xcb[1]);
    for (int k = 0; k < R; k += 2) {
      step(k, hb[0], hcb[0], xab[0], xcb[0]);
      if (k + 1 < R) step(k + 1, hb[1], hcb[1], xab[1], xcb[1]);
    }
  }

  // ---- fold lanes, then the block's waves, in a fixed order
#pragma unroll
  for (int i = 0; i < NSTAT; ++i) st[i] = ppo::wave_sum_d(st[i]);
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    db_a[j] = ppo::wave_sum(db_a[j]);
    dsc[j] = ppo::wave_sum(dsc[j]);
  }
  db_c = ppo::wave_sum(db_c);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < NSTAT; ++i) s_stats[wave][i] = st[i];
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      s_vec[wave][0][j] = db_a[j];
      s_vec[wave][2][j] = dsc[j];
    }
    s_vec[wave][1][0] = db_c;
  }
  float* fold = smem;  // [F][NA + 1]
  const int ldf = NA + 1;
  for (int w = 0; w < HL_WAVES; ++w) {
    if (wave == w) {
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        const int f = lane + 64 * e;
        if (f < F) {
#pragma unroll
          for (int j = 0; j < NA; ++j) fold[f * ldf + j] = (w ? fold[f * ldf + j] : 0.f) + acc_a[e][j];
          fold[f * ldf + NA] = (w ? fold[f * ldf + NA] : 0.f) + acc_c[e];
        }
      }
    }
    __syncthreads();
  }
  const int64_t blk = blockIdx.x;
  for (int i = threadIdx.x; i < F * (int)p.ldwa; i += HL_THREADS) {
    const int f = i / (int)p.ldwa, j = i % (int)p.ldwa;
    p.wpart_a[blk * F * p.ldwa + i] = j < NA ? fold[f * ldf + j] : 0.f;
  }
  if (SEP) {
    for (int i = threadIdx.x; i < F * (int)p.ldwc; i += HL_THREADS) {
      const int f = i / (int)p.ldwc, j = i % (int)p.ldwc;
      p.wpart_c[blk * F * p.ldwc + i] = j == 0 ? fold[f * ldf + NA] : 0.f;
    }
  }
  if (threadIdx.x < (int)p.ldwa) {
    float t = 0.f;
    for (int w = 0; w < HL_WAVES; ++w) t += threadIdx.x < NA ? s_vec[w][0][threadIdx.x] : 0.f;
    p.bpart_a[blk * p.ldwa + threadIdx.x] = t;
  }
  if (SEP && threadIdx.x < (int)p.ldwc) {
    float t = 0.f;
    for (int w = 0; w < HL_WAVES; ++w) t += threadIdx.x == 0 ? s_vec[w][1][0] : 0.f;
    p.bpart_c[blk * p.ldwc + threadIdx.x] = t;
  }
  if (p.scale_param && threadIdx.x < A) {
    float t = 0.f;
    for (int w = 0; w < HL_WAVES; ++w) t += s_vec[w][2][threadIdx.x];
    p.dscale_partial[blk * A + threadIdx.x] = t;
  }
  if (threadIdx.x < NSTAT) {
    double t = 0.0;
    for (int w = 0; w < HL_WAVES; ++w) t += s_stats[w][threadIdx.x];
    p.stats_partial[blk * NSTAT + threadIdx.x] = t;
  }
}

template <int VPL, int NA, bool SEP>
int launch(hipStream_t st, const HeadLossParams& p, int blocks) {
  const size_t shm = sizeof(float) * (size_t)p.F * (NA + 1);
  hipLaunchKernelGGL((head_loss_kernel<VPL, NA, SEP>), dim3(blocks), dim3(HL_THREADS), shm, st, p);
  return ppo::check_launch("ppo_head_loss_f32");
}

template <int VPL, bool SEP>
int launch_na(hipStream_t st, const HeadLossParams& p, int blocks) {
  if (p.na <= 4) return launch<VPL, 4, SEP>(st, p, blocks);
  if (p.na <= 8) return launch<VPL, 8, SEP>(st, p, blocks);
  return launch<VPL, 16, SEP>(st, p, blocks);
}

template <bool SEP>
int launch_vpl(hipStream_t st, const HeadLossParams& p, int blocks) {
  const int vpl = ppo::ceil_div(p.F, 64);
  if (vpl <= 1) return launch_na<1, SEP>(st, p, blocks);
  if (vpl <= 2) return launch_na<2, SEP>(st, p, blocks);
  if (vpl <= 4) return launch_na<4, SEP>(st, p, blocks);
  return launch_na<8, SEP>(st, p, blocks);
}

}  // namespace

// Blocks the fused kernel launches for `rows` (the partial buffers' leading extent).
// At least enough waves that each owns <= 64 rows; up to 512 blocks otherwise.
PPO_EXPORT int ppo_head_loss_blocks(int rows) {
  const int need = ppo::ceil_div(rows, HL_WAVES * 64);
  return std::max(std::max(1, need), std::min(ppo::ceil_div(rows, HL_WAVES * 16), 512));
}

// Largest head width (outputs of group a) and feature width the fused kernel takes.
PPO_EXPORT int ppo_head_loss_max_outputs(void) { return 16; }
PPO_EXPORT int ppo_head_loss_max_features(void) { return 512; }

PPO_EXPORT int ppo_head_loss_f32(
    void* stream, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha, const float* wa,
    int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc, int64_t ldwc,
    const float* bc, int F, int A, const float* scale_param, const int32_t* action_i, const float* action_f,
    const float* old_logp, const float* old_value, const float* adv, const float* ret, int act_a,
    const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature) {
  const bool sep = hc != nullptr;
  if (rows < 0 || F <= 0 || F > 512 || na <= 0 || na > 16 || ldwa < na || A <= 0 || A > 16 ||
      (dist != DIST_CATEGORICAL && dist != DIST_GAUSSIAN) || !ha || !wa || !ba || !old_logp || !old_value ||
      !adv || !ret || !dha || !wpart_a || !bpart_a || !stats_partial || temperature <= 0.f)
    return ppo::set_error(PPO_ERR_ARG, "ppo_head_loss_f32: bad argument (rows=%d F=%d na=%d A=%d)", rows, F, na, A);
  if (sep && (!wc || !bc || !dhc || !wpart_c || !bpart_c || ldwc < 1))
    return ppo::set_error(PPO_ERR_ARG, "ppo_head_loss_f32: separate heads need the critic buffers");
  if ((dist == DIST_CATEGORICAL && !action_i) || (dist == DIST_GAUSSIAN && !action_f))
    return ppo::set_error(PPO_ERR_ARG, "ppo_head_loss_f32: missing actions");
  if (scale_param && !dscale_partial) return ppo::set_error(PPO_ERR_ARG, "ppo_head_loss_f32: missing dscale buffer");
  if ((act_a != ACT_NONE && !aux_a) || (sep && act_c != ACT_NONE && !aux_c))
    return ppo::set_error(PPO_ERR_ARG, "ppo_head_loss_f32: activation derivative needs aux");
  if (rows == 0) return PPO_OK;
  HeadLossParams p;
  p.dist = dist; p.rows = rows; p.idx = idx;
  p.ha = ha; p.ldha = ldha; p.wa = wa; p.ldwa = ldwa; p.ba = ba; p.na = na;
  p.hc = hc; p.ldhc = ldhc; p.wc = wc; p.ldwc = ldwc; p.bc = bc;
  p.F = F; p.A = A; p.scale_param = scale_param; p.action_i = action_i; p.action_f = action_f;
  p.old_logp = old_logp; p.old_value = old_value; p.adv = adv; p.ret = ret;
  p.act_a = act_a; p.aux_a = aux_a; p.ldaux_a = ldaux_a; p.dha = dha; p.lddha = lddha;
  p.act_c = act_c; p.aux_c = aux_c; p.ldaux_c = ldaux_c; p.dhc = dhc; p.lddhc = lddhc;
  p.wpart_a = wpart_a; p.bpart_a = bpart_a; p.wpart_c = wpart_c; p.bpart_c = bpart_c;
  p.dscale_partial = dscale_partial; p.stats_partial = stats_partial;
  p.clip_eps = clip_eps; p.clip_value_loss = clip_value_loss; p.ent_coef = ent_coef; p.vf_coef = vf_coef;
  p.inv_n = 1.f / (float)rows; p.temperature = temperature;
  const int blocks = ppo_head_loss_blocks(rows);
  hipStream_t st = ppo::as_stream(stream);
  return sep ? launch_vpl<true>(st, p, blocks) : launch_vpl<false>(st, p, blocks);
}
