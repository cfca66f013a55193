// Pieces of the fused policy / value heads + PPO loss shared by the head
// loss kernels (headloss.hip) and the Gaussian torso chain that runs them on
// its last layer's output (mlp_chain.hip): the argument block, the rollout
// inputs of a (row, column) thread, and phase B, the loss and the head
// outputs' cotangents of a tile of rows (loss_fn of
// boonta/algorithms/ppo.py:77-146 with the distributions of
// boonta/networks/distributions.py:8-57).
#pragma once

#include "common.h"

namespace ppo_hl {

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
  // optional: each row's ratio exp(logp - old_logp) written env-major,
  // ratio_out[(s % ratio_envs) * ratio_steps + s / ratio_envs] for sample s = t * N + env
  float* ratio_out; int ratio_envs, ratio_steps;
  // elements between consecutive samples of old_logp, old_value, adv, ret
  // and action_i (1: separate columns); rec4: those four are one 16-byte
  // aligned float4 per sample (ppo_pack_samples records), read as one load
  int64_t sample_stride;
  bool rec4;
};

// jax's tie rule: x's share of the cotangent of ans = min / max (x, y) is 1
// when x alone is ans, 1/2 when both are (the division by 2 or 1 written as
// the exact product by 1/2 or 1).
__device__ __forceinline__ float tie_first(float x, float y, float ans) {
  return (x == ans ? 1.f : 0.f) * (y == ans ? 0.5f : 1.f);
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

// Phase B runs element-parallel: thread t owns output column j = t % 16 of
// local rows t / 16 + 16 g (g < ROWS / 16).  The 16 lanes of a row reduce
// over the head outputs with xor butterflies (every lane ends with the same
// bits: floating-point addition and max are commutative), compute the row's
// scalar loss terms redundantly, and write the row's output cotangents to
// LDS.  Block partials are column sums over the rows in LDS, in row order.

// Rollout inputs seen by one (row, column) thread of phase B; loaded at the
// start of the kernel so their latency hides behind phase A.
struct LaneIn {
  float olp, adv, ret, vold;
  float actf;  // Gaussian action component j
  int a;       // categorical action
  bool live;   // the row exists
  int64_t s;   // its sample index
};

// The rows' sample indices first (one load each), then the gathers that
// depend on them: every index load of the group is in flight before the
// first gather waits, so the chain costs two round trips, not two per row.
template <int G, int RW = 16>
__device__ __forceinline__ void lane_samples(const HeadLossParams& p, int r0, int t, LaneIn (&in)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int r = r0 + t / RW + (HL_THREADS / RW) * g;
    in[g].live = r < p.rows;
    const int rc = in[g].live ? r : p.rows - 1;
    in[g].s = p.idx ? (int64_t)p.idx[rc] : (int64_t)rc;
  }
}

template <int G>
__device__ __forceinline__ void lane_gathers(const HeadLossParams& p, int j, LaneIn (&in)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t s = in[g].s;
    const int64_t o = s * p.sample_stride;
    if (p.rec4) {
      const floatx4 r = *reinterpret_cast<const floatx4*>(p.old_logp + o);
      in[g].olp = r[0];
      in[g].vold = r[1];
      in[g].adv = r[2];
      in[g].ret = r[3];
    } else {
      in[g].olp = p.old_logp[o];
      in[g].adv = p.adv[o];
      in[g].ret = p.ret[o];
      in[g].vold = p.old_value[o];
    }
    in[g].a = 0;
    in[g].actf = 0.f;
    if (p.dist == DIST_CATEGORICAL) in[g].a = p.action_i[o];
    else in[g].actf = p.action_f[s * p.A + min(j, p.A - 1)];
  }
}

// Per-thread constants of phase B (column j): the head bias and, for a
// state-independent Gaussian scale, sigma_j, log sigma_j and the softplus
// derivative at the raw scale.
struct ColConst {
  float bias, bias_c;
  float sig, lsig, dsp;
};

__device__ __forceinline__ ColConst load_cols(const HeadLossParams& p, bool sep, int j) {
  ColConst c;
  const float b = p.ba[min(j, p.na - 1)];
  c.bias = j < p.na ? b : 0.f;
  c.bias_c = sep ? p.bc[0] : 0.f;
  c.sig = c.lsig = c.dsp = 0.f;
  if (p.scale_param) {
    const float raw = p.scale_param[min(j, p.A - 1)];
    c.sig = p.temperature * (softplusf(raw) + 1e-3f);
    c.lsig = __logf(c.sig);
    c.dsp = p.temperature / (1.f + __expf(-raw));
  }
  return c;
}

// Sum / max over a row of RW = 16 or 8 lanes (xor butterfly, every lane gets it).
template <int RW>
__device__ __forceinline__ float row_sum(float v) {
  if constexpr (RW == 16) return ppo::sum16(v);
  v += ppo::xor16<4>(v);
  v += ppo::xor16<2>(v);
  return v + ppo::xor16<1>(v);
}
template <int RW>
__device__ __forceinline__ float row_max(float v) {
  if constexpr (RW == 16) return ppo::max16(v);
  v = fmaxf(v, ppo::xor16<4>(v));
  v = fmaxf(v, ppo::xor16<2>(v));
  return fmaxf(v, ppo::xor16<1>(v));
}

// Which heads a phase B computes: both, or (separate towers run by their own
// workgroups) only the actor's or only the critic's.  The two halves are the
// same expressions as the whole, so their results are the same bits.
enum Part { PART_BOTH = 0, PART_ACTOR = 1, PART_CRITIC = 2 };

__device__ __forceinline__ constexpr bool actor_stat(int t) { return t <= ST_ADV; }

// Phase B over ROWS rows whose head outputs (no bias) are the sum of NPART
// LDS partials src[w][row][0..16] (column 16: the separate critic's value).
// Writes dout[row][0..16] (rows past the minibatch: zeros), the statistics
// and Gaussian-scale terms of each row to st / dsc, then (after a barrier)
// the block partials.  Ends with a barrier, so dout is ready for phase C.
// A row is RW = 16 lanes, or 8 for heads of at most 8 outputs (half the
// instructions: twice the rows per wave instruction; dout columns 8 .. 15
// are then written as zeros).  PART_ACTOR writes dout[row][0..16), the
// Gaussian-scale partials, the bias partials of head a and the statistics
// ST_ACTOR .. ST_ADV; PART_CRITIC dout[row][16], the bias partial of head c
// and the other statistics (SEP only).
template <int ROWS, int NPART, bool SEP, int RW = 16, int PART = PART_BOTH>
__device__ __forceinline__ void phase_b(const HeadLossParams& p, int64_t blk, const float (*src)[ROWS][LDO],
                                        float (*dout)[LDO], double (*st)[NSTAT], float (*dsc)[16],
                                        const LaneIn (&in)[ROWS * RW / HL_THREADS], const ColConst& cc) {
  static_assert(RW == 16 || RW == 8, "rows of 16 or 8 lanes");
  static_assert(PART == PART_BOTH || SEP, "one head's half needs separate heads");
  constexpr bool ACTOR = PART != PART_CRITIC, CRITIC = PART != PART_ACTOR;
  constexpr int RPG = HL_THREADS / RW;  // rows per group
  const int t = threadIdx.x;
  const int j = t % RW;
  const int A = p.A;
  const float inv_t = 1.f / p.temperature;
  const float eps = p.clip_eps;
  const bool jin = j < A;
  const bool gauss = p.dist != DIST_CATEGORICAL;
  const bool spread = p.scale_param != nullptr;
#pragma unroll
  for (int g = 0; g < ROWS / RPG; ++g) {
    const int rr = t / RW + RPG * g;
    const LaneIn& x = in[g];
    float o = 0.f;
    if (ACTOR) {
      o = src[0][rr][j];
#pragma unroll
      for (int w = 1; w < NPART; ++w) o += src[w][rr][j];
      o += cc.bias;
    }
    float v = 0.f;
    if (SEP) {
      if (CRITIC) {
        float c = src[0][rr][16];
#pragma unroll
        for (int w = 1; w < NPART; ++w) c += src[w][rr][16];
        v = c + cc.bias_c;
      }
    } else {
      v = __shfl(o, p.na - 1, RW);
    }
    float lp = 0.f, ent = 0.f, val = 0.f, draw = 0.f, pmin_r = 0.f, clip_r = 0.f, ratio_r = 0.f;
    if (ACTOR && !gauss) {
      const float z = o * inv_t;
      const float mx = row_max<RW>(jin ? z : -INFINITY);
      const float se = row_sum<RW>(jin ? __expf(z - mx) : 0.f);
      const float lse = mx + __logf(se);
      const float za = row_sum<RW>(j == x.a ? z : 0.f);
      lp = (x.a >= 0 && x.a < A) ? za - lse : -INFINITY;
      const float lq = z - lse;
      const float q = __expf(lq);
      ent = -row_sum<RW>(jin ? q * lq : 0.f);
      // per-row terms below need lp and ent; the cotangent follows them
      val = 0.f;
      const float ratio = __expf(lp - x.olp);
      float cr, dcr;
      clip_grad(ratio, 1.f - eps, 1.f + eps, cr, dcr);
      const float pg1 = ratio * x.adv, pg2 = cr * x.adv;
      const float pmin = fminf(pg1, pg2);
      const float g_lp =
          -(tie_first(pg1, pg2, pmin) * x.adv + tie_first(pg2, pg1, pmin) * x.adv * dcr) * p.inv_n * ratio;
      const float g_ent = -p.ent_coef * p.inv_n;
      val = jin ? (g_lp * ((j == x.a ? 1.f : 0.f) - q) - g_ent * q * (lq + ent)) * inv_t : 0.f;
      pmin_r = pmin;
      clip_r = (fabsf(ratio - 1.f) > eps) ? 1.f : 0.f;
      ratio_r = ratio;
    } else if (ACTOR) {
      const float raw = spread ? 0.f : __shfl(o, min(A + j, RW - 1), RW);
      const float sig = spread ? cc.sig : p.temperature * (softplusf(raw) + 1e-3f);
      const float ls = spread ? cc.lsig : __logf(sig);
      const float d = x.actf - o;
      const float zz = d / sig;
      lp = row_sum<RW>(jin ? -0.5f * zz * zz - ls - 0.5f * LOG_2PI : 0.f);
      ent = row_sum<RW>(jin ? 0.5f + 0.5f * LOG_2PI + ls : 0.f);
      const float ratio = __expf(lp - x.olp);
      float cr, dcr;
      clip_grad(ratio, 1.f - eps, 1.f + eps, cr, dcr);
      const float pg1 = ratio * x.adv, pg2 = cr * x.adv;
      const float pmin = fminf(pg1, pg2);
      const float g_lp =
          -(tie_first(pg1, pg2, pmin) * x.adv + tie_first(pg2, pg1, pmin) * x.adv * dcr) * p.inv_n * ratio;
      const float g_ent = -p.ent_coef * p.inv_n;
      val = jin ? g_lp * d / (sig * sig) : 0.f;
      const float dsig = g_lp * (d * d / (sig * sig * sig) - 1.f / sig) + g_ent / sig;
      draw = dsig * (spread ? cc.dsp : p.temperature / (1.f + __expf(-raw)));
      if (!spread) {
        const float dr = __shfl(draw, max(j - A, 0), RW);
        if (j >= A && j < 2 * A) val = dr;
      }
      pmin_r = pmin;
      clip_r = (fabsf(ratio - 1.f) > eps) ? 1.f : 0.f;
      ratio_r = ratio;
    }
    // value loss (the same in every lane of the row)
    float crow = 0.f, dvalue = 0.f;
    if (CRITIC) {
      const float vl1 = 0.5f * (v - x.ret) * (v - x.ret);
      float gv;
      if (p.clip_value_loss) {
        float dv, ddv;
        clip_grad(v - x.vold, -eps, eps, dv, ddv);
        const float vc = x.vold + dv;
        const float vl2 = 0.5f * (vc - x.ret) * (vc - x.ret);
        crow = fmaxf(vl1, vl2);
        gv = tie_first(vl1, vl2, crow) * (v - x.ret) + tie_first(vl2, vl1, crow) * (vc - x.ret) * ddv;
      } else {
        crow = vl1;
        gv = v - x.ret;
      }
      dvalue = p.vf_coef * gv * p.inv_n;
    }
    if (!SEP && j == p.na - 1) val = dvalue;
    if (ACTOR) {
      dout[rr][j] = x.live ? val : 0.f;
      if (RW == 8) dout[rr][j + 8] = 0.f;
      if (spread) dsc[rr][j] = (x.live && jin) ? draw : 0.f;
    }
    if (j == 0) {
      const bool l = x.live;
      if (CRITIC) {
        dout[rr][16] = l ? dvalue : 0.f;
        const double res = (double)x.ret - (double)v;
        st[rr][ST_CRITIC] = l ? (double)crow : 0.0;
        st[rr][ST_RESID] = l ? res : 0.0;
        st[rr][ST_RESID2] = l ? res * res : 0.0;
        st[rr][ST_RET] = l ? (double)x.ret : 0.0;
        st[rr][ST_RET2] = l ? (double)x.ret * (double)x.ret : 0.0;
        st[rr][ST_VALUE] = l ? (double)v : 0.0;
      }
      if (ACTOR) {
        st[rr][ST_ACTOR] = l ? (double)(-pmin_r) : 0.0;
        st[rr][ST_ENTROPY] = l ? (double)ent : 0.0;
        st[rr][ST_KL] = l ? (double)(x.olp - lp) : 0.0;
        st[rr][ST_CLIPFRAC] = l ? (double)clip_r : 0.0;
        st[rr][ST_ADV] = l ? (double)x.adv : 0.0;
        if (p.ratio_out && l) p.ratio_out[(x.s % p.ratio_envs) * p.ratio_steps + x.s / p.ratio_envs] = ratio_r;
      }
    }
  }
  __syncthreads();
  // block partials: column sums over the rows in row order (wave 0)
  if (t < NSTAT) {
    if (actor_stat(t) ? ACTOR : CRITIC) {
      double a = 0.0;
      for (int r = 0; r < ROWS; ++r) a += st[r][t];
      p.stats_partial[blk * NSTAT + t] = a;
    }
  } else if (t >= 16 && t < 16 + (int)p.ldwa) {
    if (ACTOR) {
      float a = 0.f;
      for (int r = 0; r < ROWS; ++r) a += dout[r][t - 16];
      p.bpart_a[blk * p.ldwa + (t - 16)] = a;
    }
  } else if (SEP && t >= 32 && t < 32 + (int)p.ldwc) {
    if (CRITIC) {
      float a = 0.f;
      if (t == 32)
        for (int r = 0; r < ROWS; ++r) a += dout[r][16];
      p.bpart_c[blk * p.ldwc + (t - 32)] = a;
    }
  } else if (spread && t >= 48 && t < 48 + A) {
    if (ACTOR) {
      float a = 0.f;
      for (int r = 0; r < ROWS; ++r) a += dsc[r][t - 48];
      p.dscale_partial[blk * A + (t - 48)] = a;
    }
  }
}

__device__ __forceinline__ floatx4 mfma4(floatx4 a, const float (&b)[4], floatx4 acc) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
  return acc;
}

// The torso activation's derivative with the activation a compile-time
// constant where the launch knows it (ACT >= 0: both towers' activation), so
// the per-element loops of phase C hold only its code; ACT < 0 switches on
// the run-time value.
template <int ACT>
__device__ __forceinline__ bool has_act(int act) { return (ACT >= 0 ? ACT : act) != ACT_NONE; }
template <int ACT>
__device__ __forceinline__ float dact(int act, float x) { return ppo::act_grad(ACT >= 0 ? ACT : act, x); }

// Checks the arguments of ppo_head_loss_f32 (messages under `name`) and fills
// p; PPO_OK, or the error code set.
int head_loss_setup(HeadLossParams& p, const char* name, int dist, int rows, const int32_t* idx, const float* ha,
                    int64_t ldha, const float* wa, int64_t ldwa, const float* ba, int na, const float* hc,
                    int64_t ldhc, const float* wc, int64_t ldwc, const float* bc, int F, int A,
                    const float* scale_param, const int32_t* action_i, const float* action_f, const float* old_logp,
                    const float* old_value, const float* adv, const float* ret, int act_a, const float* aux_a,
                    int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c, int64_t ldaux_c,
                    float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
                    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss,
                    float ent_coef, float vf_coef, float temperature, float* ratio_out, int ratio_envs,
                    int ratio_steps, int64_t sample_stride);

}  // namespace ppo_hl
