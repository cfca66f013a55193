// Fused policy/value heads + PPO loss + head backward over one minibatch.
//
// Follows loss_fn of boonta/algorithms/ppo.py:77-146 (recurrent_ppo.py:101-184)
// with the heads of boonta/networks/heads.py:9-45 (a Dense layer each, or one
// Dense feeding both when actor and critic share the torso) and the
// distributions of boonta/networks/distributions.py:8-57.
//
// One workgroup of 4 wave64s owns a tile of 64 minibatch rows and does the
// head algebra on matrix cores (v_mfma_f32_16x16x4f32), with every operand
// loaded in one pass so the global-load latency is paid a few times per tile
// rather than once per row:
//   A. head outputs OUT[64, 16] = H[64, F] Wa[F, 16] (each wave 16 rows; the
//      value of separate towers is one more column from Hc wc) -> LDS;
//   B. one lane per row: the loss, its statistics and the cotangents of the
//      head outputs (jax's tie rules for min / max / clip) -> LDS, with the
//      block's statistic, bias and Gaussian-scale partials;
//   C1. the cotangent of each head input, dH[64, F] = dOUT[64, 16] Wa^T times
//      the derivative of the torso's last activation (each wave 16 rows);
//   C2. the head weight gradient partial H^T dOUT [F, 16] (16-feature blocks
//      dealt round-robin to the waves).
// Every loop issues the loads of four 16-wide steps before their MFMAs, so
// four global round trips overlap.
// Per-block partials are summed in a fixed order by the gradient reduce, so
// results do not depend on scheduling.  F must be a multiple of 16 (<= 512)
// and the heads have at most 16 outputs.
#include "common.h"

#include <algorithm>

namespace {

constexpr int HL_THREADS = 256;

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


constexpr int TR = 64;   // rows per workgroup
constexpr int LDO = 20;  // LDS row pitch: 16 head outputs + the separate critic's value, 16-byte rows

// The loss and output cotangents of one row (phase B).  out[0..15]: head
// outputs with bias; v: the value.  Writes dout[0..15], dvalue and adds to
// the statistics / Gaussian-scale accumulators.
__device__ __forceinline__ void row_loss(const HeadLossParams& p, bool sep, int64_t s, const float (&out)[16],
                                         float v, float (&dout)[16], float& dvalue, double (&st)[NSTAT],
                                         float (&dsc)[16]) {
  const int A = p.A;
  const float olp = p.old_logp[s], Av = p.adv[s], Rt = p.ret[s], vold = p.old_value[s];
  const float eps = p.clip_eps;
  const float inv_t = 1.f / p.temperature;
  float lp = 0.f, ent = 0.f, lse = 0.f;
  int a = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) dout[j] = 0.f;
  if (p.dist == DIST_CATEGORICAL) {
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) if (j < A) mx = fmaxf(mx, out[j] * inv_t);
    float se = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) if (j < A) se += __expf(out[j] * inv_t - mx);
    lse = mx + __logf(se);
    a = p.action_i[s];
    float za = -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) za = (j == a) ? out[j] * inv_t : za;
    lp = (a >= 0 && a < A) ? za - lse : -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < A) {
        const float lq = out[j] * inv_t - lse;
        ent -= __expf(lq) * lq;
      }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < A) {
        float raw = 0.f;
        if (p.scale_param) {
          raw = p.scale_param[j];
        } else {
#pragma unroll
          for (int q = 0; q < 16; ++q) raw = (q == A + j) ? out[q] : raw;
        }
        const float sig = p.temperature * (softplusf(raw) + 1e-3f);
        const float zz = (p.action_f[s * A + j] - out[j]) / sig;
        const float ls = __logf(sig);
        lp += -0.5f * zz * zz - ls - 0.5f * LOG_2PI;
        ent += 0.5f + 0.5f * LOG_2PI + ls;
      }
  }
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
  dvalue = p.vf_coef * gv * p.inv_n;
  if (p.dist == DIST_CATEGORICAL) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < A) {
        const float lq = out[j] * inv_t - lse;
        const float q = __expf(lq);
        dout[j] = (g_lp * ((j == a ? 1.f : 0.f) - q) - g_ent * q * (lq + ent)) * inv_t;
      }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < A) {
        float raw = 0.f;
        if (p.scale_param) {
          raw = p.scale_param[j];
        } else {
#pragma unroll
          for (int q = 0; q < 16; ++q) raw = (q == A + j) ? out[q] : raw;
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
          for (int q = 0; q < 16; ++q) dout[q] = (q == A + j) ? draw : dout[q];
        }
      }
  }
  if (!sep) {
#pragma unroll
    for (int j = 0; j < 16; ++j) dout[j] = (j == p.na - 1) ? dvalue : dout[j];
  }
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

__device__ __forceinline__ floatx4 mfma4(floatx4 a, const float (&b)[4], floatx4 acc) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
  return acc;
}

template <bool SEP>
__global__ void __launch_bounds__(HL_THREADS) head_loss_kernel(HeadLossParams p) {
  __shared__ __attribute__((aligned(16))) float s_out[TR][LDO];
  __shared__ __attribute__((aligned(16))) float s_dout[TR][LDO];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;   // MFMA row (A) / column (B, D)
  const int kq = lane >> 4;   // MFMA k group; D rows 4 * kq + v
  const int F = p.F;
  const int r0 = blockIdx.x * TR;
  const int64_t blk = blockIdx.x;

  // ---------------- A. head outputs of the wave's 16 rows
  {
    const int row = r0 + 16 * wave + li;
    const bool live = row < p.rows;
    const float* hrow = p.ha + (int64_t)(live ? row : 0) * p.ldha;
    const float* crow = SEP ? p.hc + (int64_t)(live ? row : 0) * p.ldhc : nullptr;
    const bool jv = li < p.na;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f}, accc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < F; k0 += 64) {
      floatx4 av[4], cv[4];
      float bv[4][4], wv[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int k = k0 + 16 * u + 4 * kq;
        const bool in = live && k0 + 16 * u < F;
        av[u] = in ? *reinterpret_cast<const floatx4*>(hrow + k) : floatx4{0.f, 0.f, 0.f, 0.f};
        if (SEP) cv[u] = in ? *reinterpret_cast<const floatx4*>(crow + k) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bool kin = k0 + 16 * u < F;
          bv[u][s] = (jv && kin) ? p.wa[(int64_t)(k + s) * p.ldwa + li] : 0.f;
          if (SEP) wv[u][s] = (li == 0 && kin) ? p.wc[(int64_t)(k + s) * p.ldwc] : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc = mfma4(av[u], bv[u], acc);
        if (SEP) accc = mfma4(cv[u], wv[u], accc);
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      s_out[16 * wave + 4 * kq + v][li] = acc[v];
      if (SEP && li == 0) s_out[16 * wave + 4 * kq + v][16] = accc[v];
    }
  }
  __syncthreads();

  // ---------------- B. loss and output cotangents, one lane of wave 0 per row
  if (wave == 0) {
    double st[NSTAT];
#pragma unroll
    for (int i = 0; i < NSTAT; ++i) st[i] = 0.0;
    float db[16], dsc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) db[j] = dsc[j] = 0.f;
    float dbc = 0.f;
    const int r = r0 + lane;
    float dout[16];
    float dvalue = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) dout[j] = 0.f;
    if (r < p.rows) {
      const int64_t s = p.idx ? (int64_t)p.idx[r] : (int64_t)r;
      float out[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) out[j] = s_out[lane][j] + (j < p.na ? p.ba[j] : 0.f);
      const float v = SEP ? s_out[lane][16] + p.bc[0] : out[p.na - 1];
      row_loss(p, SEP, s, out, v, dout, dvalue, st, dsc);
#pragma unroll
      for (int j = 0; j < 16; ++j) db[j] = dout[j];
      dbc = dvalue;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) s_dout[lane][j] = dout[j];
    s_dout[lane][16] = dvalue;
    // block partials: statistics, head biases, Gaussian scale (fixed-order wave sums)
#pragma unroll
    for (int i = 0; i < NSTAT; ++i) st[i] = ppo::wave_sum_d(st[i]);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      db[j] = ppo::wave_sum(db[j]);
      dsc[j] = ppo::wave_sum(dsc[j]);
    }
    dbc = ppo::wave_sum(dbc);
    if (lane < NSTAT) {
      double t = 0.0;
#pragma unroll
      for (int i = 0; i < NSTAT; ++i) t = (i == lane) ? st[i] : t;
      p.stats_partial[blk * NSTAT + lane] = t;
    }
    if (lane < (int)p.ldwa) {
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) t = (j == lane) ? db[j] : t;
      p.bpart_a[blk * p.ldwa + lane] = t;
    }
    if (SEP && lane < (int)p.ldwc) p.bpart_c[blk * p.ldwc + lane] = lane == 0 ? dbc : 0.f;
    if (p.scale_param && lane < p.A) {
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) t = (j == lane) ? dsc[j] : t;
      p.dscale_partial[blk * p.A + lane] = t;
    }
  }
  __syncthreads();

  // ---------------- C1. cotangent of the head inputs (the wave's 16 rows)
  {
    const floatx4 dv4 = *reinterpret_cast<const floatx4*>(&s_dout[16 * wave + li][4 * kq]);
    const bool live_a = r0 + 16 * wave + li < p.rows;
    const floatx4 a_in = live_a ? dv4 : floatx4{0.f, 0.f, 0.f, 0.f};
    for (int f0 = 0; f0 < F; f0 += 64) {
      float bv[4][4], xa[4][4], xc[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int f = f0 + 16 * u + li;  // B column = output feature
        const bool fin = f0 + 16 * u < F;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int j = 4 * kq + s;
          bv[u][s] = (fin && j < p.na) ? p.wa[(int64_t)f * p.ldwa + j] : 0.f;
          const int row = r0 + 16 * wave + 4 * kq + s;
          const bool ok = fin && row < p.rows;
          xa[u][s] = (ok && p.act_a != ACT_NONE) ? p.aux_a[(int64_t)row * p.ldaux_a + f] : 0.f;
          if (SEP) xc[u][s] = (ok && p.act_c != ACT_NONE) ? p.aux_c[(int64_t)row * p.ldaux_c + f] : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int f = f0 + 16 * u + li;
        if (f0 + 16 * u >= F) break;
        const floatx4 g = mfma4(a_in, bv[u], floatx4{0.f, 0.f, 0.f, 0.f});
        const float wcf = SEP ? p.wc[(int64_t)f * p.ldwc] : 0.f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int rr = 16 * wave + 4 * kq + v;
          const int row = r0 + rr;
          if (row >= p.rows) continue;
          float d = g[v];
          if (p.act_a != ACT_NONE) d *= ppo::act_grad(p.act_a, xa[u][v]);
          p.dha[(int64_t)row * p.lddha + f] = d;
          if (SEP) {
            float dc = s_dout[rr][16] * wcf;
            if (p.act_c != ACT_NONE) dc *= ppo::act_grad(p.act_c, xc[u][v]);
            p.dhc[(int64_t)row * p.lddhc + f] = dc;
          }
        }
      }
    }
  }

  // ---------------- C2. head weight gradient partial H^T dOUT (16-feature blocks dealt to the waves)
  {
    for (int fb = 16 * wave; fb < F; fb += 64) {
      const int f = fb + li;  // A row = feature
      floatx4 acc = {0.f, 0.f, 0.f, 0.f}, accc = {0.f, 0.f, 0.f, 0.f};
      floatx4 av[TR / 16], cv[TR / 16];
#pragma unroll
      for (int cc = 0; cc < TR / 16; ++cc) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int row = r0 + 16 * cc + 4 * kq + s;
          const bool ok = row < p.rows;
          av[cc][s] = ok ? p.ha[(int64_t)row * p.ldha + f] : 0.f;
          cv[cc][s] = (SEP && ok) ? p.hc[(int64_t)row * p.ldhc + f] : 0.f;
        }
      }
#pragma unroll
      for (int cc = 0; cc < TR / 16; ++cc) {
        float bv[4], wv[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int rr = 16 * cc + 4 * kq + s;
          bv[s] = s_dout[rr][li];
          wv[s] = (SEP && li == 0) ? s_dout[rr][16] : 0.f;
        }
        acc = mfma4(av[cc], bv, acc);
        if (SEP) accc = mfma4(cv[cc], wv, accc);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int ff = fb + 4 * kq + v;
        if (li < (int)p.ldwa) p.wpart_a[(blk * F + ff) * p.ldwa + li] = acc[v];
        if (SEP && li < (int)p.ldwc) p.wpart_c[(blk * F + ff) * p.ldwc + li] = li == 0 ? accc[v] : 0.f;
      }
    }
  }
}

}  // namespace

// Blocks the fused kernel launches for `rows` (the partial buffers' leading
// extent): one per 64-row tile.
PPO_EXPORT int ppo_head_loss_blocks(int rows) { return std::max(1, ppo::ceil_div(rows, TR)); }

// Largest head width (outputs of group a) and feature width the fused kernel
// takes; the feature width must also be a multiple of 16.
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
  if (rows < 0 || F <= 0 || F > 512 || F % 16 != 0 || na <= 0 || na > 16 || ldwa < na || ldwa > 16 || A <= 0 ||
      A > 16 ||
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
  if (sep && ldwc > 16) return ppo::set_error(PPO_ERR_ARG, "ppo_head_loss_f32: ldwc > 16");
  if ((reinterpret_cast<uintptr_t>(ha) & 15) || ldha % 4 || (sep && ((reinterpret_cast<uintptr_t>(hc) & 15) || ldhc % 4)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_head_loss_f32: head inputs need 16-byte aligned rows");
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
  if (sep) hipLaunchKernelGGL(head_loss_kernel<true>, dim3(blocks), dim3(HL_THREADS), 0, st, p);
  else hipLaunchKernelGGL(head_loss_kernel<false>, dim3(blocks), dim3(HL_THREADS), 0, st, p);
  return ppo::check_launch("ppo_head_loss_f32");
}
