// Row-wise kernels of the learner: LayerNorm (+activation) forward/backward,
// standalone activations, and the fused PPO loss with its gradient.
//
// LayerNorm follows flax 0.12.8 LayerNorm as composed by the configs
// (epsilon 1e-6, fast variance E[x^2] - E[x]^2 clipped at 0, statistics in
// fp32, learned scale and bias).  One wavefront owns one row; the feature
// axis (<= 1024) sits across the 64 lanes, so statistics are wave reductions.
//
// The loss follows boonta/algorithms/ppo.py:77-146 (recurrent_ppo.py:101-184)
// and the distributions of boonta/networks/distributions.py:8-57.  It takes
// the head outputs (logits, or Gaussian mean / raw scale, and the value) of one
// minibatch, and writes the cotangents of those outputs, the per-block partial
// sums behind the 8 logged scalars (ppo.py:167-180), and for a
// state-independent Gaussian scale its gradient partials.  One lane owns one
// sample; the head width is small (<= 64).
#include "common.h"

namespace {

constexpr int ROW_THREADS = 256;
constexpr int MAX_VPL = 16;  // features per lane: F <= 1024

// ------------------------------------------------------------ LayerNorm fwd
// z [rows, F] (ld ldz) -> y = act(LN(z)) [rows, F] (ld ldy); mean/rstd [rows].
// ACT: the activation (a compile-time constant: the element loops then hold
// only its code; the act argument is the same value).
template <int VPL, int ACT>
__global__ void __launch_bounds__(ROW_THREADS)
ln_act_fwd_kernel(const float* __restrict__ z, int64_t ldz, const float* __restrict__ gamma,
                  const float* __restrict__ beta, float* __restrict__ y, int64_t ldy, float* __restrict__ mean_out,
                  float* __restrict__ rstd_out, int rows, int F, float eps, int act, int round,
                  uint16_t* __restrict__ y16, int64_t ldy16) {
  const int lane = threadIdx.x & 63;
  const int wpb = ROW_THREADS / 64;
  for (int64_t r = (int64_t)blockIdx.x * wpb + (threadIdx.x >> 6); r < rows; r += (int64_t)gridDim.x * wpb) {
    const float* zr = z + r * ldz;
    float v[VPL];
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      const int f = lane + 64 * e;
      v[e] = f < F ? zr[f] : 0.f;
    }
    float mean, rstd;
    ppo::ln_row_stats<VPL>(v, (float)F, eps, mean, rstd);
    if (lane == 0) {
      if (mean_out) mean_out[r] = mean;
      if (rstd_out) rstd_out[r] = rstd;
    }
    float* yr = y ? y + r * ldy : nullptr;
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      const int f = lane + 64 * e;
      if (f < F) {
        float o = ppo::ln_row_apply(v[e], mean, rstd, gamma[f], beta[f]);
        if (round) {
          // flax casts the fp32 LayerNorm result back to the bf16 compute dtype
          o = ppo::bf16_round(o);
          o = ppo::act_fwd(ACT, o);
          if (ACT != ACT_RELU && ACT != ACT_NONE) o = ppo::bf16_round(o);
        } else {
          o = ppo::act_fwd(ACT, o);
        }
        if (yr) yr[f] = o;
        if (y16) y16[r * ldy16 + f] = (uint16_t)ppo::bf16_bits(o);
      }
    }
  }
}

// ------------------------------------------------------------ LayerNorm bwd
// Element strides of tower t's buffers in a tower-batched launch (blockIdx.y
// = tower): dy / z / dz rows, mean / rstd, gamma / beta, and the partials.
struct LnTowers {
  int64_t rows, stats, params, part;
};

// dy = dL/d(act output) [rows, F]; recomputes the LN output from z, mean,
// rstd; writes dz [rows, F] and per-block partials [gridDim.x][2F] holding
// (sum over the block's rows of dyl * xhat | sum of dyl) for scale and bias.
template <int VPL, int ACT>
__global__ void __launch_bounds__(ROW_THREADS)
ln_act_bwd_kernel(const float* __restrict__ dy, int64_t lddy, const float* __restrict__ z, int64_t ldz,
                  const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
                  const float* __restrict__ gamma, const float* __restrict__ beta, void* __restrict__ dz,
                  int64_t lddz, float* __restrict__ partial, int rows, int F, int act, int round, int out16,
                  LnTowers tw) {
#pragma clang fp contract(off)  // the roundings of ppo::ln_bwd_dyl / ln_bwd_dz's callers stay as written
  if (blockIdx.y) {  // tower t of a tower-batched launch
    const int64_t t = blockIdx.y;
    dy += t * tw.rows;
    z += t * tw.rows;
    dz = static_cast<float*>(dz) + t * tw.rows;
    mean_in += t * tw.stats;
    rstd_in += t * tw.stats;
    gamma += t * tw.params;
    beta += t * tw.params;
    partial += t * tw.part;
  }
  __shared__ float red[ROW_THREADS / 64][2][VPL * 64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wpb = ROW_THREADS / 64;
  float acc_g[VPL], acc_b[VPL], gam[VPL], bet[VPL];
#pragma unroll
  for (int e = 0; e < VPL; ++e) {
    acc_g[e] = acc_b[e] = 0.f;
    const int f = lane + 64 * e;
    gam[e] = f < F ? gamma[f] : 0.f;
    bet[e] = f < F ? beta[f] : 0.f;
  }
  // A wave takes rows r0, r0 + stride, ... and loads RB of them before
  // computing any, so their global-load latencies overlap.
  constexpr int RB = VPL <= 8 ? 4 : 2;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  for (int64_t r0 = (int64_t)blockIdx.x * wpb + wave; r0 < rows; r0 += RB * stride) {
    float zv[RB][VPL], dv[RB][VPL], mu[RB], rs[RB];
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int64_t r = r0 + j * stride;
      const int64_t rr = r < rows ? r : r0;
      mu[j] = mean_in[rr];
      rs[j] = rstd_in[rr];
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        const int f = lane + 64 * e;
        const int fc = f < F ? f : 0;
        zv[j][e] = z[rr * ldz + fc];
        dv[j][e] = dy[rr * lddy + fc];
      }
    }
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int64_t r = r0 + j * stride;
      if (r >= rows) break;
      const float mean = mu[j];
      const float rstd = rs[j];
      float xh[VPL], g[VPL];
      float sg = 0.f, sgx = 0.f;
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        const int f = lane + 64 * e;
        if (f < F) {
          const float dyl = ppo::ln_bwd_dyl<ACT>(zv[j][e], dv[j][e], mean, rstd, gam[e], bet[e], round, xh[e]);
          acc_g[e] = __fmaf_rn(dyl, xh[e], acc_g[e]);
          acc_b[e] += dyl;
          g[e] = dyl * gam[e];
        } else {
          xh[e] = 0.f;
          g[e] = 0.f;
        }
        sg += g[e];
        sgx = __fmaf_rn(g[e], xh[e], sgx);
      }
      sg = ppo::wave_sum(sg) / (float)F;
      sgx = ppo::wave_sum(sgx) / (float)F;
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        const int f = lane + 64 * e;
        if (f < F) {
          const float d = ppo::ln_bwd_dz(g[e], xh[e], sg, sgx, rstd);
          if (out16)
            static_cast<uint16_t*>(dz)[r * lddz + f] = (uint16_t)ppo::bf16_bits(d);
          else
            static_cast<float*>(dz)[r * lddz + f] = round ? ppo::bf16_round(d) : d;
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < VPL; ++e) {
    red[wave][0][lane + 64 * e] = acc_g[e];
    red[wave][1][lane + 64 * e] = acc_b[e];
  }
  __syncthreads();
  for (int f = threadIdx.x; f < F; f += ROW_THREADS) {
    float sgm = 0.f, sb = 0.f;
#pragma unroll
    for (int w = 0; w < wpb; ++w) {
      sgm += red[w][0][f];
      sb += red[w][1][f];
    }
    partial[(int64_t)blockIdx.x * 2 * F + f] = sgm;
    partial[(int64_t)blockIdx.x * 2 * F + F + f] = sb;
  }
}

// ------------------------------------------------------------- activations
__global__ void act_fwd_kernel(const float* __restrict__ x, int64_t ldx, float* __restrict__ y, int64_t ldy,
                               int rows, int F, int act) {
  const int64_t total = (int64_t)rows * F;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / F, f = i % F;
    y[r * ldy + f] = ppo::act_fwd(act, x[r * ldx + f]);
  }
}

// dx = dy * act'(aux): aux is the activation output (relu, tanh) or input (silu)
__global__ void act_bwd_kernel(const float* __restrict__ dy, int64_t lddy, const float* __restrict__ aux,
                               int64_t ldaux, float* __restrict__ dx, int64_t lddx, int rows, int F, int act) {
  const int64_t total = (int64_t)rows * F;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / F, f = i % F;
    dx[r * lddx + f] = dy[r * lddy + f] * ppo::act_grad(act, aux[r * ldaux + f]);
  }
}

// -------------------------------------------------------------------- loss
enum Dist { DIST_CATEGORICAL = 0, DIST_GAUSSIAN = 1 };

// Statistic slots of the per-block partial sums (doubles).
enum Stat {
  ST_ACTOR = 0,    // sum of -min(r A, clip(r) A)
  ST_ENTROPY,      // sum of entropy
  ST_KL,           // sum of old_logp - logp
  ST_CLIPFRAC,     // count of |r - 1| > eps
  ST_ADV,          // sum of A
  ST_CRITIC,       // sum of the (clipped) value loss rows
  ST_RESID,        // sum of (R - v)
  ST_RESID2,       // sum of (R - v)^2
  ST_RET,          // sum of R
  ST_RET2,         // sum of R^2
  ST_VALUE,        // sum of v
  NSTAT
};

struct LossParams {
  int dist;
  int rows;
  const int32_t* idx;  // minibatch row -> sample index (null: identity)
  // head outputs of the minibatch
  const float* head;  // logits [rows, A] or Gaussian mean [rows, D] (+ raw scale at +D when state-dependent)
  int64_t ldh;
  const float* value;  // value at value[r * ldv]
  int64_t ldv;
  int A;                      // categories, or Gaussian dimension D
  const float* scale_param;   // state-independent raw Gaussian scale [D] or null
  // per-sample inputs (indexed by idx)
  const int32_t* action_i;   // categorical actions [B]
  const float* action_f;     // Gaussian actions [B, D]
  const float* old_logp;
  const float* old_value;
  const float* adv;
  const float* ret;
  // outputs
  float* dhead;  // same layout as head
  float* dvalue;
  float* dscale_partial;  // [gridDim.x][D] or null
  double* stats_partial;  // [gridDim.x][NSTAT]
  // hyper-parameters
  float clip_eps;
  int clip_value_loss;
  float ent_coef;
  float vf_coef;
  float inv_n;
  float temperature;
};

// jax's cotangent split for min/max at a tie, and jnp.clip = min(hi, max(lo, x))
__device__ __forceinline__ float tie_first(float x, float y, float ans) {
  return (x == ans ? 1.f : 0.f) / (y == ans ? 2.f : 1.f);
}
__device__ __forceinline__ void clip_grad(float x, float lo, float hi, float& out, float& dx) {
  const float m = fmaxf(lo, x);
  const float dm = tie_first(x, lo, m);
  out = fminf(hi, m);
  dx = tie_first(m, hi, out) * dm;
}

__device__ __forceinline__ float softplusf(float x) {
  // log(1 + e^x) without overflow
  return fmaxf(x, 0.f) + log1pf(__expf(-fabsf(x)));
}

constexpr float LOG_2PI = 1.8378770664093453f;

// One 16-lane group per row: lane j0 of the group owns head outputs j0,
// j0 + 16, ... (A <= 64); the row's log-softmax or log-density and entropy are
// 16-lane butterflies, the scalar clip and value terms are evaluated by every
// lane of the group alike, and lane 0 of the group adds the row to the block's
// statistics.  Rows are walked in block-sized strides; a group whose row is
// past the end idles through the iteration (its butterflies stay inside it).
constexpr int LOSS_THREADS = 256;
constexpr int LOSS_GROUP = 16;
constexpr int LOSS_ROWS = LOSS_THREADS / LOSS_GROUP;
constexpr int LOSS_K = 4;  // head outputs per lane

static_assert(LOSS_GROUP == 16, "the group reductions are 16-lane DPP butterflies");
__device__ __forceinline__ float group16_sum(float v) { return ppo::sum16(v); }
__device__ __forceinline__ float group16_max(float v) { return ppo::max16(v); }

__global__ void __launch_bounds__(LOSS_THREADS) ppo_loss_kernel(LossParams p) {
  __shared__ double sred[LOSS_THREADS / 64][NSTAT];
  __shared__ float sscale[LOSS_THREADS / 64][LOSS_GROUP];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j0 = threadIdx.x % LOSS_GROUP;
  const int grow = threadIdx.x / LOSS_GROUP;
  double st[NSTAT];
#pragma unroll
  for (int i = 0; i < NSTAT; ++i) st[i] = 0.0;
  float dscale_acc = 0.f;  // state-independent scale: output j0 (D <= 16)
  const float eps = p.clip_eps;
  const float inv_t = 1.f / p.temperature;

  for (int r0 = blockIdx.x * LOSS_ROWS; r0 < p.rows; r0 += gridDim.x * LOSS_ROWS) {
    const int r = r0 + grow;
    if (r >= p.rows) continue;
    const int64_t s = p.idx ? (int64_t)p.idx[r] : (int64_t)r;
    const float* hr = p.head + (int64_t)r * p.ldh;
    float* dr = p.dhead + (int64_t)r * p.ldh;
    float lp, ent;
    float c[LOSS_K];
    float lse = 0.f;
    int a = -1;
    if (p.dist == DIST_CATEGORICAL) {
      float mx = -INFINITY;
#pragma unroll
      for (int k = 0; k < LOSS_K; ++k) {
        const int j = j0 + LOSS_GROUP * k;
        c[k] = j < p.A ? hr[j] * inv_t : -INFINITY;
        mx = fmaxf(mx, c[k]);
      }
      mx = group16_max(mx);
      float se = 0.f;
#pragma unroll
      for (int k = 0; k < LOSS_K; ++k)
        if (j0 + LOSS_GROUP * k < p.A) se += __expf(c[k] - mx);
      lse = mx + __logf(group16_sum(se));
      a = p.action_i[s];
      float lpa = 0.f, en = 0.f;
#pragma unroll
      for (int k = 0; k < LOSS_K; ++k) {
        const int j = j0 + LOSS_GROUP * k;
        if (j < p.A) {
          const float lq = c[k] - lse;
          if (j == a) lpa = lq;
          en -= __expf(lq) * lq;
        }
      }
      // distrax: log_prob of a value outside [0, A) is -inf
      const float lpsum = group16_sum(lpa);
      lp = (a >= 0 && a < p.A) ? lpsum : -INFINITY;
      ent = group16_sum(en);
    } else {
      float l = 0.f, e = 0.f;
      const float* act = p.action_f + s * p.A;
#pragma unroll
      for (int k = 0; k < LOSS_K; ++k) {
        const int j = j0 + LOSS_GROUP * k;
        if (j < p.A) {
          const float raw = p.scale_param ? p.scale_param[j] : hr[p.A + j];
          const float sig = p.temperature * (softplusf(raw) + 1e-3f);
          const float zz = (act[j] - hr[j]) / sig;
          const float ls = __logf(sig);
          l += -0.5f * zz * zz - ls - 0.5f * LOG_2PI;
          e += 0.5f + 0.5f * LOG_2PI + ls;
        }
      }
      lp = group16_sum(l);
      ent = group16_sum(e);
    }
    const float olp = p.old_logp[s];
    const float A = p.adv[s];
    const float R = p.ret[s];
    const float vold = p.old_value[s];
    const float v = p.value[(int64_t)r * p.ldv];

    // actor: -min(r A, clip(r, 1-eps, 1+eps) A)
    const float ratio = __expf(lp - olp);
    float cr, dcr;
    clip_grad(ratio, 1.f - eps, 1.f + eps, cr, dcr);
    const float pg1 = ratio * A, pg2 = cr * A;
    const float pmin = fminf(pg1, pg2);
    const float d_ratio = -(tie_first(pg1, pg2, pmin) * A + tie_first(pg2, pg1, pmin) * A * dcr) * p.inv_n;
    const float g_lp = d_ratio * ratio;
    const float g_ent = -p.ent_coef * p.inv_n;

    // critic: max(0.5 (v - R)^2, 0.5 (v_old + clip(v - v_old, -eps, eps) - R)^2)
    const float vl1 = 0.5f * (v - R) * (v - R);
    float crow, gv;
    if (p.clip_value_loss) {
      float dv, ddv;
      clip_grad(v - vold, -eps, eps, dv, ddv);
      const float vc = vold + dv;
      const float vl2 = 0.5f * (vc - R) * (vc - R);
      crow = fmaxf(vl1, vl2);
      gv = tie_first(vl1, vl2, crow) * (v - R) + tie_first(vl2, vl1, crow) * (vc - R) * ddv;
    } else {
      crow = vl1;
      gv = v - R;
    }
    if (j0 == 0) p.dvalue[(int64_t)r * p.ldv] = p.vf_coef * gv * p.inv_n;

    // cotangents of the head outputs
    if (p.dist == DIST_CATEGORICAL) {
#pragma unroll
      for (int k = 0; k < LOSS_K; ++k) {
        const int j = j0 + LOSS_GROUP * k;
        if (j < p.A) {
          const float lq = c[k] - lse;
          const float q = __expf(lq);
          const float d = g_lp * ((j == a ? 1.f : 0.f) - q) - g_ent * q * (lq + ent);
          dr[j] = d * inv_t;
        }
      }
    } else {
      const float* act = p.action_f + s * p.A;
#pragma unroll
      for (int k = 0; k < LOSS_K; ++k) {
        const int j = j0 + LOSS_GROUP * k;
        if (j < p.A) {
          const float raw = p.scale_param ? p.scale_param[j] : hr[p.A + j];
          const float sp = softplusf(raw);
          const float sig = p.temperature * (sp + 1e-3f);
          const float d = act[j] - hr[j];
          dr[j] = g_lp * d / (sig * sig);
          const float dsig = g_lp * (d * d / (sig * sig * sig) - 1.f / sig) + g_ent / sig;
          const float draw = dsig * p.temperature / (1.f + __expf(-raw));
          if (p.scale_param) {
            dscale_acc += draw;  // k = 0: D <= 16
          } else {
            dr[p.A + j] = draw;
          }
        }
      }
    }

    if (j0 == 0) {
      st[ST_ACTOR] += (double)(-pmin);
      st[ST_ENTROPY] += (double)ent;
      st[ST_KL] += (double)(olp - lp);
      st[ST_CLIPFRAC] += (fabsf(ratio - 1.f) > eps) ? 1.0 : 0.0;
      st[ST_ADV] += (double)A;
      st[ST_CRITIC] += (double)crow;
      const double res = (double)R - (double)v;
      st[ST_RESID] += res;
      st[ST_RESID2] += res * res;
      st[ST_RET] += (double)R;
      st[ST_RET2] += (double)R * (double)R;
      st[ST_VALUE] += (double)v;
    }
  }

#pragma unroll
  for (int i = 0; i < NSTAT; ++i) {
    const double t = ppo::wave_sum_d(st[i]);
    if (lane == 0) sred[wave][i] = t;
  }
  if (p.scale_param) {
    // the wave's four groups hold the same outputs: fold them, lanes 0-15 keep the sums
    float v = dscale_acc;
    v = ppo::add_xor16(v);
    v = ppo::add_xor32(v);
    if (lane < LOSS_GROUP) sscale[wave][lane] = v;
  }
  __syncthreads();
  if (threadIdx.x < NSTAT) {
    double t = 0.0;
    for (int w = 0; w < LOSS_THREADS / 64; ++w) t += sred[w][threadIdx.x];
    p.stats_partial[(int64_t)blockIdx.x * NSTAT + threadIdx.x] = t;
  }
  if (p.scale_param && threadIdx.x < p.A) {
    float t = 0.f;
    for (int w = 0; w < LOSS_THREADS / 64; ++w) t += sscale[w][threadIdx.x];
    p.dscale_partial[(int64_t)blockIdx.x * p.A + threadIdx.x] = t;
  }
}

// Folds the per-block partial sums into the 8 logged scalars of one minibatch
// step (ppo.py:170-179 order): actor/loss, actor/entropy, actor/approximate_kl,
// actor/clip_fraction, actor/advantage, critic/loss, critic/explained_variance,
// critic/value; then the total loss in slot 8.
__global__ void __launch_bounds__(256)
loss_finalize_kernel(const double* __restrict__ partial, int nblocks, int rows, float ent_coef, float vf_coef,
                     float* __restrict__ out) {
  __shared__ double s[NSTAT];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // block i finalizes step i: partials [steps][nblocks][NSTAT], out [steps][9]
  partial += (int64_t)blockIdx.x * nblocks * NSTAT;
  out += (int64_t)blockIdx.x * 9;
  // wave w folds statistics w, w + 4, w + 8 over the block partials
  for (int k = wave; k < NSTAT; k += 4) {
    double t = 0.0;
    for (int b = lane; b < nblocks; b += 64) t += partial[(int64_t)b * NSTAT + k];
    t = ppo::wave_sum_d(t);
    if (lane == 0) s[k] = t;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const double n = (double)rows;
    const double actor = s[ST_ACTOR] / n, entropy = s[ST_ENTROPY] / n, critic = s[ST_CRITIC] / n;
    const double mr = s[ST_RESID] / n, mR = s[ST_RET] / n;
    const double var_res = fmax(s[ST_RESID2] / n - mr * mr, 0.0);
    const double var_ret = fmax(s[ST_RET2] / n - mR * mR, 0.0);
    out[0] = (float)actor;
    out[1] = (float)entropy;
    out[2] = (float)(s[ST_KL] / n);
    out[3] = (float)(s[ST_CLIPFRAC] / n);
    out[4] = (float)(s[ST_ADV] / n);
    out[5] = (float)critic;
    out[6] = (float)(1.0 - var_res / (var_ret + 1e-8));
    out[7] = (float)(s[ST_VALUE] / n);
    out[8] = (float)(actor - (double)ent_coef * entropy + (double)vf_coef * critic);
  }
}

template <int VPL>
int launch_ln_fwd(hipStream_t st, int blocks, const float* z, int64_t ldz, const float* gamma, const float* beta,
                  float* y, int64_t ldy, float* mean, float* rstd, int rows, int F, float eps, int act, int round,
                  uint16_t* y16, int64_t ldy16) {
#define PPO_LN_FWD(A)                                                                                   \
  hipLaunchKernelGGL((ln_act_fwd_kernel<VPL, A>), dim3(blocks), dim3(ROW_THREADS), 0, st, z, ldz, gamma, beta, y, ldy, \
                     mean, rstd, rows, F, eps, act, round, y16, ldy16)
  switch (act) {
    case ACT_RELU: PPO_LN_FWD(ACT_RELU); break;
    case ACT_TANH: PPO_LN_FWD(ACT_TANH); break;
    case ACT_SILU: PPO_LN_FWD(ACT_SILU); break;
    default: PPO_LN_FWD(ACT_NONE); break;
  }
#undef PPO_LN_FWD
  return ppo::check_launch("ppo_layernorm_act_fwd_f32");
}

template <int VPL>
int launch_ln_bwd(hipStream_t st, int blocks, const float* dy, int64_t lddy, const float* z, int64_t ldz,
                  const float* mean, const float* rstd, const float* gamma, const float* beta, void* dz,
                  int64_t lddz, float* partial, int rows, int F, int act, int round, int out16, int towers,
                  LnTowers tw) {
#define PPO_LN_BWD(A)                                                                                       \
  hipLaunchKernelGGL((ln_act_bwd_kernel<VPL, A>), dim3(blocks, towers), dim3(ROW_THREADS), 0, st, dy, lddy, z, ldz, \
                     mean, rstd, gamma, beta, dz, lddz, partial, rows, F, act, round, out16, tw)
  switch (act) {
    case ACT_RELU: PPO_LN_BWD(ACT_RELU); break;
    case ACT_TANH: PPO_LN_BWD(ACT_TANH); break;
    case ACT_SILU: PPO_LN_BWD(ACT_SILU); break;
    default: PPO_LN_BWD(ACT_NONE); break;
  }
#undef PPO_LN_BWD
  return ppo::check_launch("ppo_layernorm_act_bwd_f32");
}

}  // namespace

static int layernorm_fwd(const char* name, void* stream, const float* z, int64_t ldz, const float* gamma,
                         const float* beta, float* y, int64_t ldy, float* mean, float* rstd, int rows, int F,
                         float eps, int act, int round, uint16_t* y16 = nullptr, int64_t ldy16 = 0) {
  // y may be NULL only when the bf16 copy y16 is written (the fp32 output unused)
  if (rows < 0 || F <= 0 || F > 64 * MAX_VPL || act < 0 || act > 3 || !z || !gamma || !beta || (!y && !y16))
    return ppo::set_error(PPO_ERR_ARG, "%s: bad argument (rows=%d F=%d)", name, rows, F);
  if (rows == 0) return PPO_OK;
  const int blocks = std::min(ppo::ceil_div(rows, ROW_THREADS / 64), 4096);
  hipStream_t st = ppo::as_stream(stream);
  const int vpl = ppo::ceil_div(F, 64);
  if (vpl <= 1) return launch_ln_fwd<1>(st, blocks, z, ldz, gamma, beta, y, ldy, mean, rstd, rows, F, eps, act, round, y16, ldy16);
  if (vpl <= 2) return launch_ln_fwd<2>(st, blocks, z, ldz, gamma, beta, y, ldy, mean, rstd, rows, F, eps, act, round, y16, ldy16);
  if (vpl <= 4) return launch_ln_fwd<4>(st, blocks, z, ldz, gamma, beta, y, ldy, mean, rstd, rows, F, eps, act, round, y16, ldy16);
  if (vpl <= 8) return launch_ln_fwd<8>(st, blocks, z, ldz, gamma, beta, y, ldy, mean, rstd, rows, F, eps, act, round, y16, ldy16);
  return launch_ln_fwd<16>(st, blocks, z, ldz, gamma, beta, y, ldy, mean, rstd, rows, F, eps, act, round, y16, ldy16);
}

PPO_EXPORT int ppo_layernorm_act_fwd_f32(void* stream, const float* z, int64_t ldz, const float* gamma,
                                         const float* beta, float* y, int64_t ldy, float* mean, float* rstd,
                                         int rows, int F, float eps, int act) {
  return layernorm_fwd("ppo_layernorm_act_fwd_f32", stream, z, ldz, gamma, beta, y, ldy, mean, rstd, rows, F, eps,
                       act, 0);
}

// bf16 compute: statistics and normalisation in fp32, the result rounded to bf16.
PPO_EXPORT int ppo_layernorm_act_fwd_bf16(void* stream, const float* z, int64_t ldz, const float* gamma,
                                          const float* beta, float* y, int64_t ldy, float* mean, float* rstd,
                                          int rows, int F, float eps, int act) {
  return layernorm_fwd("ppo_layernorm_act_fwd_bf16", stream, z, ldz, gamma, beta, y, ldy, mean, rstd, rows, F, eps,
                       act, 1);
}

// The same, also storing the output as bf16 bit patterns (y16, row pitch
// ldy16 elements): the bf16 operand of the next layer's GEMMs.
PPO_EXPORT int ppo_layernorm_act_fwd_bf16_out16(void* stream, const float* z, int64_t ldz, const float* gamma,
                                                const float* beta, float* y, int64_t ldy, void* y16, int64_t ldy16,
                                                float* mean, float* rstd, int rows, int F, float eps, int act) {
  if (!y16 || ldy16 < F) return ppo::set_error(PPO_ERR_ARG, "ppo_layernorm_act_fwd_bf16_out16: bad bf16 output");
  return layernorm_fwd("ppo_layernorm_act_fwd_bf16_out16", stream, z, ldz, gamma, beta, y, ldy, mean, rstd, rows, F,
                       eps, act, 1, static_cast<uint16_t*>(y16), ldy16);
}

// Partials: [blocks][2F]; blocks = ppo_layernorm_bwd_blocks(rows).
PPO_EXPORT int ppo_layernorm_bwd_blocks(int rows) {
  // two rows per wave until the grid holds 512 blocks (more rows per wave beyond)
  return std::max(1, std::min(ppo::ceil_div(rows, 2 * (ROW_THREADS / 64)), 512));
}

static int layernorm_bwd(const char* name, void* stream, const float* dy, int64_t lddy, const float* z,
                         int64_t ldz, const float* mean, const float* rstd, const float* gamma, const float* beta,
                         void* dz, int64_t lddz, float* partial, int rows, int F, int act, int round,
                         int out16 = 0, int towers = 1, LnTowers tw = LnTowers{0, 0, 0, 0}) {
  if (rows < 0 || F <= 0 || F > 64 * MAX_VPL || act < 0 || act > 3 || !dy || !z || !mean || !rstd || !gamma ||
      !beta || !dz || !partial || towers < 1 || towers > 8 || (towers > 1 && out16))
    return ppo::set_error(PPO_ERR_ARG, "%s: bad argument (rows=%d F=%d)", name, rows, F);
  const int blocks = ppo_layernorm_bwd_blocks(rows);
  hipStream_t st = ppo::as_stream(stream);
  const int vpl = ppo::ceil_div(F, 64);
  if (vpl <= 1) return launch_ln_bwd<1>(st, blocks, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz, lddz, partial, rows, F, act, round, out16,
                                            towers, tw);
  if (vpl <= 2) return launch_ln_bwd<2>(st, blocks, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz, lddz, partial, rows, F, act, round, out16,
                                            towers, tw);
  if (vpl <= 4) return launch_ln_bwd<4>(st, blocks, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz, lddz, partial, rows, F, act, round, out16,
                                            towers, tw);
  if (vpl <= 8) return launch_ln_bwd<8>(st, blocks, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz, lddz, partial, rows, F, act, round, out16,
                                            towers, tw);
  return launch_ln_bwd<16>(st, blocks, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz, lddz, partial, rows, F, act, round, out16,
                                            towers, tw);
}

PPO_EXPORT int ppo_layernorm_act_bwd_f32(void* stream, const float* dy, int64_t lddy, const float* z, int64_t ldz,
                                         const float* mean, const float* rstd, const float* gamma,
                                         const float* beta, float* dz, int64_t lddz, float* partial, int rows,
                                         int F, int act) {
  return layernorm_bwd("ppo_layernorm_act_bwd_f32", stream, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz, lddz,
                       partial, rows, F, act, 0);
}

// ppo_layernorm_act_bwd_f32 over `towers` layers of one shape in one grid:
// tower t's dy / z / dz rows, mean / rstd, gamma / beta and partials sit t
// times the given element strides after tower 0's.
PPO_EXPORT int ppo_layernorm_act_bwd_f32_towers(void* stream, int towers, const float* dy, int64_t lddy,
                                                const float* z, int64_t ldz, const float* mean, const float* rstd,
                                                const float* gamma, const float* beta, float* dz, int64_t lddz,
                                                float* partial, int rows, int F, int act, int64_t stride_rows,
                                                int64_t stride_stats, int64_t stride_params, int64_t stride_part) {
  return layernorm_bwd("ppo_layernorm_act_bwd_f32_towers", stream, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz,
                       lddz, partial, rows, F, act, 0, 0, towers,
                       LnTowers{stride_rows, stride_stats, stride_params, stride_part});
}

// bf16 compute: the LayerNorm output was rounded to bf16 before the activation,
// and the input cotangent is rounded to bf16 (the cast's transpose).
PPO_EXPORT int ppo_layernorm_act_bwd_bf16(void* stream, const float* dy, int64_t lddy, const float* z, int64_t ldz,
                                          const float* mean, const float* rstd, const float* gamma,
                                          const float* beta, float* dz, int64_t lddz, float* partial, int rows,
                                          int F, int act) {
  return layernorm_bwd("ppo_layernorm_act_bwd_bf16", stream, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz, lddz,
                       partial, rows, F, act, 1);
}

// The same with the input cotangent stored as bf16 bit patterns (dz16, row
// pitch lddz16 elements): the bf16 operand of the first layer's dW GEMM.
PPO_EXPORT int ppo_layernorm_act_bwd_bf16_out16(void* stream, const float* dy, int64_t lddy, const float* z,
                                                int64_t ldz, const float* mean, const float* rstd,
                                                const float* gamma, const float* beta, void* dz16, int64_t lddz16,
                                                float* partial, int rows, int F, int act) {
  return layernorm_bwd("ppo_layernorm_act_bwd_bf16_out16", stream, dy, lddy, z, ldz, mean, rstd, gamma, beta, dz16,
                       lddz16, partial, rows, F, act, 1, 1);
}

PPO_EXPORT int ppo_act_fwd_f32(void* stream, const float* x, int64_t ldx, float* y, int64_t ldy, int rows, int F,
                               int act) {
  if (rows < 0 || F < 0 || act < 0 || act > 3 || !x || !y)
    return ppo::set_error(PPO_ERR_ARG, "ppo_act_fwd_f32: bad argument");
  if (rows == 0 || F == 0) return PPO_OK;
  const int blocks = (int)std::min<int64_t>(ppo::ceil_div64((int64_t)rows * F, 256), 8192);
  hipLaunchKernelGGL(act_fwd_kernel, dim3(blocks), dim3(256), 0, ppo::as_stream(stream), x, ldx, y, ldy, rows, F, act);
  return ppo::check_launch("ppo_act_fwd_f32");
}

PPO_EXPORT int ppo_act_bwd_f32(void* stream, const float* dy, int64_t lddy, const float* aux, int64_t ldaux,
                               float* dx, int64_t lddx, int rows, int F, int act) {
  if (rows < 0 || F < 0 || act < 0 || act > 3 || !dy || !aux || !dx)
    return ppo::set_error(PPO_ERR_ARG, "ppo_act_bwd_f32: bad argument");
  if (rows == 0 || F == 0) return PPO_OK;
  const int blocks = (int)std::min<int64_t>(ppo::ceil_div64((int64_t)rows * F, 256), 8192);
  hipLaunchKernelGGL(act_bwd_kernel, dim3(blocks), dim3(256), 0, ppo::as_stream(stream), dy, lddy, aux, ldaux, dx,
                     lddx, rows, F, act);
  return ppo::check_launch("ppo_act_bwd_f32");
}

PPO_EXPORT int ppo_loss_blocks(int rows) {
  return std::max(1, std::min(ppo::ceil_div(rows, LOSS_ROWS), 1024));
}

PPO_EXPORT int ppo_loss_stat_count(void) { return NSTAT; }

// Fused PPO loss + head-output cotangents for one minibatch (see LossParams).
PPO_EXPORT int ppo_loss_f32(void* stream, int dist, int rows, const int32_t* idx, const float* head, int64_t ldh,
                            const float* value, int64_t ldv, int A, const float* scale_param,
                            const int32_t* action_i, const float* action_f, const float* old_logp,
                            const float* old_value, const float* adv, const float* ret, float* dhead,
                            float* dvalue, float* dscale_partial, double* stats_partial, float clip_eps,
                            int clip_value_loss, float ent_coef, float vf_coef, float temperature) {
  if (rows < 0 || A <= 0 || A > 64 || (dist != DIST_CATEGORICAL && dist != DIST_GAUSSIAN) || !head || !value ||
      !old_logp || !old_value || !adv || !ret || !dhead || !dvalue || !stats_partial || temperature <= 0.f)
    return ppo::set_error(PPO_ERR_ARG, "ppo_loss_f32: bad argument (rows=%d A=%d dist=%d)", rows, A, dist);
  if (dist == DIST_CATEGORICAL && !action_i) return ppo::set_error(PPO_ERR_ARG, "ppo_loss_f32: missing actions");
  if (dist == DIST_GAUSSIAN && !action_f) return ppo::set_error(PPO_ERR_ARG, "ppo_loss_f32: missing actions");
  if (scale_param && (A > 16 || !dscale_partial))
    return ppo::set_error(PPO_ERR_ARG, "ppo_loss_f32: state-independent scale needs D <= 16 and a partial buffer");
  if (rows == 0) return PPO_OK;
  LossParams p;
  p.dist = dist; p.rows = rows; p.idx = idx; p.head = head; p.ldh = ldh; p.value = value; p.ldv = ldv; p.A = A;
  p.scale_param = scale_param; p.action_i = action_i; p.action_f = action_f; p.old_logp = old_logp;
  p.old_value = old_value; p.adv = adv; p.ret = ret; p.dhead = dhead; p.dvalue = dvalue;
  p.dscale_partial = dscale_partial; p.stats_partial = stats_partial; p.clip_eps = clip_eps;
  p.clip_value_loss = clip_value_loss; p.ent_coef = ent_coef; p.vf_coef = vf_coef; p.inv_n = 1.f / (float)rows;
  p.temperature = temperature;
  hipLaunchKernelGGL(ppo_loss_kernel, dim3(ppo_loss_blocks(rows)), dim3(LOSS_THREADS), 0, ppo::as_stream(stream), p);
  return ppo::check_launch("ppo_loss_f32");
}

PPO_EXPORT int ppo_loss_finalize_steps(void* stream, const double* stats_partial, int nblocks, int rows, int steps,
                                       float ent_coef, float vf_coef, float* out) {
  if (nblocks <= 0 || rows <= 0 || steps < 0 || (steps > 0 && (!stats_partial || !out)))
    return ppo::set_error(PPO_ERR_ARG, "ppo_loss_finalize_steps: bad argument");
  if (steps == 0) return PPO_OK;
  hipLaunchKernelGGL(loss_finalize_kernel, dim3(steps), dim3(256), 0, ppo::as_stream(stream), stats_partial, nblocks,
                     rows, ent_coef, vf_coef, out);
  return ppo::check_launch("ppo_loss_finalize_steps");
}

PPO_EXPORT int ppo_loss_finalize(void* stream, const double* stats_partial, int nblocks, int rows, float ent_coef,
                                 float vf_coef, float* out9) {
  if (nblocks <= 0 || rows <= 0 || !stats_partial || !out9)
    return ppo::set_error(PPO_ERR_ARG, "ppo_loss_finalize: bad argument");
  hipLaunchKernelGGL(loss_finalize_kernel, dim3(1), dim3(256), 0, ppo::as_stream(stream), stats_partial, nblocks,
                     rows, ent_coef, vf_coef, out9);
  return ppo::check_launch("ppo_loss_finalize");
}
