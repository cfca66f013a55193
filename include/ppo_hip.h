/*
 * libppo_hip.so — C ABI of the MI355X (gfx950) PPO learner kernels.
 *
 * These are the entry points the XLA FFI custom-call targets of boonta's
 * learner bind (one handler per target, each forwarding XLA's stream and
 * buffers to the launcher below).  They take a HIP stream
 * as `void*`, device pointers and sizes; enqueue work asynchronously; never
 * synchronise, allocate, or retain pointers across calls; and return 0 or a
 * negative status, with a message from ppo_last_error() on the calling thread.
 * Every [T, N] array is time-major (row t, column n), as boonta's rollout
 * leaves it; every matrix is row-major with an explicit leading dimension.
 */
#ifndef PPO_HIP_H_
#define PPO_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define PPO_OK 0
#define PPO_ERR_ARG (-1)
#define PPO_ERR_LAUNCH (-2)
#define PPO_ERR_SPACE (-3)

/* Activation codes (flax.linen relu / tanh / silu). */
#define PPO_ACT_NONE 0
#define PPO_ACT_RELU 1
#define PPO_ACT_TANH 2
#define PPO_ACT_SILU 3

/* Distribution codes of the actor head. */
#define PPO_DIST_CATEGORICAL 0
#define PPO_DIST_GAUSSIAN 1

/* ---------------------------------------------------------------- errors */
const char* ppo_last_error(void);
void ppo_clear_error(void);
int ppo_abi_version(void);
int ppo_device_check(int device);
/* Stream ordering for running independent chains (the actor and critic
 * towers) on two streams: ppo_stream_wait makes work issued on `waiter`
 * after the call start after everything issued on `signaller` before it
 * (event recorded on signaller, waited on by waiter; inside a stream capture
 * this forks / joins the graph).  Streams are hipStream_t handles. */
int ppo_event_create(void** event);
int ppo_event_destroy(void* event);
int ppo_stream_wait(void* waiter, void* signaller, void* event);

/* ------------------------------------------------------------------- GAE
 * Replaces boonta/algorithms/advantage_estimators.py:8-56
 * (generalized_advantage_estimator(transitions, values, bootstrap, gamma,
 * gae_lambda, rho=1., c=1.) -> (advantages, returns)), called at
 * boonta/algorithms/ppo.py:213-219 and recurrent_ppo.py:199-205.
 * reward/values/rho/c/advantages/returns: float [T, N]; terminated/truncated:
 * bool bytes [T, N]; bootstrap: float [N]; rho, c may be NULL (= 1).
 * chunks: pieces the T axis is cut into (<= 16); 0 picks one. */
int ppo_gae_f32(void* stream, const float* reward, const uint8_t* terminated, const uint8_t* truncated,
                const float* values, const float* bootstrap, const float* rho, const float* c,
                float* advantages, float* returns, int T, int N, double gamma, double gae_lambda,
                int chunks);

/* V-trace (boonta/algorithms/recurrent_pupo.py:210-220: the estimator above
 * with rho = min(ratio, advantage_clip), c = min(ratio, trace_clip)); ratio
 * is float [N, T] env-major with row pitch ldr >= T, moved to time-major as
 * the reference's jnp.moveaxis does, by indexing. */
int ppo_vtrace_f32(void* stream, const float* reward, const uint8_t* terminated, const uint8_t* truncated,
                   const float* values, const float* bootstrap, const float* ratio, int64_t ldr, float advantage_clip,
                   float trace_clip, float* advantages, float* returns, int T, int N, double gamma, double gae_lambda,
                   int chunks);

/* Advantage normalisation (A - mean) / (std + 1e-8), population std over
 * all n advantages, in place: boonta/algorithms/ppo.py:220-221 and
 * recurrent_ppo.py:206-207 (PPOConfig.normalize_advantage). */
size_t ppo_normalize_workspace(int64_t n);
int ppo_normalize_advantages_f32(void* stream, float* adv, int64_t n, void* workspace, size_t workspace_bytes);

/* RecurrentPuPO's minibatch advantages (boonta/algorithms/recurrent_pupo.py:
 * 244-250): out[rows[i]] = weights[i % width] * A'[i] where A' is advantages
 * [rows[i]] normalised over the count = T * width minibatch samples when
 * normalize ((A - mean) / (std + 1e-8), population std), rows[i] = t * N + env
 * listed time-major (ppo_sequence_rows), weights [width] the importance weight
 * of each drawn sequence (ppo_priority_choice_f32). */
int ppo_pupo_advantages_f32(void* stream, const float* advantages, const int32_t* rows, int count,
                            const float* weights, int width, int normalize, float* out);
/* a[i] = value for i < n (a fill that a captured graph can hold; RecurrentPuPO
 * starts every update from ratio = ones, recurrent_pupo.py:306). */
int ppo_fill_f32(void* stream, float* a, int64_t n, float value);

/* ----------------------------------------------------------- permutation
 * Replace jax.random.split(key, E) and jax.random.permutation(key, n) at
 * boonta/algorithms/ppo.py:200,230 and recurrent_ppo.py:272,278 (jax 0.10.2,
 * threefry2x32, partitionable).  key: device uint32[2] key data. */
int ppo_threefry_split(void* stream, const uint32_t* key, uint32_t* out, int64_t num);
size_t ppo_permutation_workspace(int64_t n);
/* The bucket sort's plan for n items (host only, no launch): the bucket count
 * is 2^ppo_permutation_bucket_bits(n); buckets of up to
 * ppo_permutation_bucket_cap(n) items are sorted in LDS, larger ones (not
 * expected below 2^24 items) are ranked from global memory. */
int ppo_permutation_bucket_bits(int64_t n);
int ppo_permutation_bucket_cap(int64_t n);
int ppo_permutation(void* stream, const uint32_t* key, int32_t* out, int64_t n, void* workspace,
                    size_t workspace_bytes);
size_t ppo_epoch_permutations_workspace(int epochs, int64_t n);
/* out[e * n + i] = permutation(split(key, epochs)[e], n)[i] (ppo.py:199-201,230-231). */
int ppo_epoch_permutations(void* stream, const uint32_t* key, int epochs, int64_t n, int32_t* out,
                           void* workspace, size_t workspace_bytes);
/* No counterpart in the reference.  ppo_epoch_permutations for callers that
 * cannot allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc): the same results, with the workspace in the library's own
 * 24 MiB device scratch (one per GPU, held until the process ends) instead of
 * an argument.  Returns PPO_ERR_SPACE when ppo_epoch_permutations_workspace
 * (epochs, n) exceeds 24 MiB (4 epochs of 262144 items need 20.5 MiB), and
 * PPO_ERR_ARG when the stream's device is not the current device.  Calls that
 * overlap on one GPU share the scratch and race: order them on one stream. */
int ppo_epoch_permutations_noalloc(void* stream, const uint32_t* key, int epochs, int64_t n, int32_t* out);

/* -------------------------------------------------------------- sampling
 * Replace dist.sample_and_log_prob(seed=key) in the rollout-side PPO.step
 * (boonta/algorithms/ppo.py:57-74) for boonta's categorical head
 * (networks/distributions.py:8-23: log_softmax of preferences / temperature,
 * Gumbel-max draw of jax.random.gumbel(key, (1, rows, A)), greedy one-hot at
 * temperature <= 0) and diagonal Gaussian head (distributions.py:42-57:
 * sigma = temperature * (softplus(s) + 1e-3), eps = jax.random.normal(key,
 * (1, rows, D)), action = sigma * eps + mean).  key: device uint32[2] key data,
 * used as given (no split).  value (may be NULL) receives value_src[r * ldv],
 * the critic column (remove_feature_axis, utils/axis.py:11-12).  A and D are at
 * most ppo_sample_max_outputs(). */
int ppo_sample_max_outputs(void);
int ppo_sample_categorical_f32(void* stream, const float* pref, int64_t ldp, int rows, int A,
                               const float* value_src, int64_t ldv, const uint32_t* key, float temperature,
                               int32_t* action, float* log_prob, float* value);
/* scale_raw: the raw scale s, [rows, lds] per row (state-dependent head: the
 * second half of the head outputs), or one [D] vector when lds == 0
 * (state-independent SpreadScale parameter). */
int ppo_sample_gaussian_f32(void* stream, const float* mean, int64_t ldm, const float* scale_raw, int64_t lds,
                            int rows, int D, const float* value_src, int64_t ldv, const uint32_t* key,
                            float temperature, float* action, int64_t lda, float* log_prob, float* value);

/* The whole PPO.step (boonta/algorithms/ppo.py:57-74) of a shared-trunk MLP
 * with a categorical head in one launch: `layers` trunk Dense layers of 256
 * features with one activation (network.py:18-49, MLP torso,
 * networks/blocks/mlp.py), the shared head Dense [256, ldwh] whose columns
 * 0..A-1 are the logits and column A the value (ActorCritic head), and the
 * categorical draw of ppo_sample_categorical_f32.  weights / ldw / biases are
 * HOST arrays of `layers` entries (device pointers to 16-byte aligned
 * [K_l, 256] kernels, ldw[l] == 256; K_0 = obs_dim, K_l = 256 after); ldwh <= 16.
 * Same outputs as the trunk GEMMs, the head GEMM and the sampling launch. */
int ppo_step_mlp_max_layers(void);
int ppo_step_mlp_max_obs(void); /* obs_dim limit (the rows are staged in LDS) */
int ppo_step_mlp_categorical_f32(void* stream, const float* obs, int64_t ldo, int rows, int obs_dim, int layers,
                                 const float* const* weights, const int64_t* ldw, const float* const* biases, int act,
                                 const float* head_w, int64_t ldwh, const float* head_b, int A, const uint32_t* key,
                                 float temperature, int32_t* action, float* log_prob, float* value);

/* --------------------------------------------- prioritised env selection
 * Replaces the minibatch selection of RecurrentPuPO.update
 * (boonta/algorithms/recurrent_pupo.py:226-236): priority[n] =
 * (sum_t |advantages[t, n]|) ** priority_exponent, probabilities[n] =
 * (priority[n] + 1e-6) / (sum priority + 1e-6), indices =
 * jax.random.choice(key, N, (width,), replace=True, p=probabilities) (inverse
 * CDF on the key's uniform stream), weights[i] = (N * probabilities[indices[i]])
 * ** -beta.  advantages: float [T, N] with row pitch lda (the V-trace output of
 * ppo_gae_f32 with rho = min(ratio, advantage_clip), c = min(ratio,
 * trace_clip)); indices int32 [width]; weights float [width]; probabilities
 * float [N] (required).  N <= ppo_priority_choice_max_envs().  The draws search
 * a float64 running sum of the float32 probabilities; jax types that sum and
 * r in float32.  Against a float32 sequential cumsum the indices agree on
 * every draw at 1024 envs drawing 256 and differ, by one env, on at most 0.6 %
 * of draws up to 16384 envs (22 of 4096). */
int ppo_priority_choice_max_envs(void);
int ppo_priority_choice_f32(void* stream, const float* advantages, int64_t lda, int T, int N, float priority_exponent,
                            float beta, const uint32_t* key, int width, int32_t* indices, float* weights,
                            float* probabilities);

/* ------------------------------------------------ Dense + LayerNorm + act
 * One torso layer of flax Dense -> LayerNorm -> activation (the Gaussian
 * workload's towers, hangar recipes' 4 x 256 SiLU MLPs) in a single launch:
 * Z = X W + b (row r of X is X[rows_idx[r]] when rows_idx is non-NULL), the
 * row statistics of Z (fast variance, as flax's LayerNorm) and
 * Y = act((Z - mean) rstd gamma + beta).  Writes Z, mean, rstd and Y, the same
 * values ppo_gemm_f32 (epi 1, no activation) followed by
 * ppo_layernorm_act_fwd_f32 leave.  F must be 256. */
int ppo_gemm_ln_act_fwd_f32(void* stream, const float* X, int64_t ldx, const int32_t* rows_idx, const float* W,
                            int64_t ldw, const float* bias, const float* gamma, const float* beta, float* Z,
                            int64_t ldz, float* Y, int64_t ldy, float* mean, float* rstd, int M, int K, int F,
                            float eps, int act);
/* The same layer for `towers` (<= 8) towers of one shape in one grid (the
 * actor and critic towers of flax's ActorCritic with separate torsos, one
 * launch per depth instead of two): tower t reads X + t stride_x (0 when the
 * towers read the same rows), its W / bias / gamma / beta at
 * + t stride_params, and writes Z and Y at + t stride_rows and mean / rstd at
 * + t stride_stats (elements; stride_x, stride_params and stride_rows
 * multiples of 4).  Bit-identical to one ppo_gemm_ln_act_fwd_f32 per tower. */
int ppo_gemm_ln_act_fwd_f32_towers(void* stream, int towers, const float* X, int64_t ldx, const int32_t* rows_idx,
                                   const float* W, int64_t ldw, const float* bias, const float* gamma,
                                   const float* beta, float* Z, int64_t ldz, float* Y, int64_t ldy, float* mean,
                                   float* rstd, int M, int K, int F, float eps, int act, int64_t stride_x,
                                   int64_t stride_params, int64_t stride_rows, int64_t stride_stats);

/* ------------------------------------------------- whole torso chains
 * The actor and critic towers of flax's ActorCritic with separate torsos
 * of L (<= ppo_mlp_chain_max_layers()) Dense(256) -> LayerNorm -> activation
 * layers (boonta/networks/network.py:38-49; the backward of
 * jax.value_and_grad at boonta/algorithms/ppo.py:155-157), every layer of
 * every tower in one launch per direction: rows are independent through the
 * torso, so each 16-row workgroup runs the chain with the activations in
 * LDS or registers.  Array arguments hold tower 0's per-layer pointers;
 * tower t's buffers sit t times the given element strides after them
 * (multiples of 4, towers <= 8).
 *
 * Forward: layer 0 reads X (row r = X[rows_idx[r]] when rows_idx is
 * non-NULL; K0 features, kernel [K0][ldw0]), layer l > 0 the previous
 * output (kernel [256][ldw], ldw == 256); each layer writes Z = x W + b, its row mean /
 * rstd (fast variance) and Y = act(LayerNorm(Z)).  Bit-identical to one
 * ppo_gemm_ln_act_fwd_f32 per layer.  WT (may be NULL): for l >= 1, WT[l]
 * receives layer l's kernel transposed ([256 out][256 in], pitch 256; tower
 * t's at t * stride_wt), the operand ppo_mlp_ln_bwd_f32 reads. */
int ppo_mlp_chain_max_layers(void);
int ppo_mlp_ln_fwd_f32(void* stream, int towers, int L, const float* X, int64_t ldx, const int32_t* rows_idx, int M,
                       int K0, const float* const* W, int64_t ldw0, int64_t ldw, const float* const* bias,
                       const float* const* gamma, const float* const* beta, float* const* Z, float* const* Y,
                       int64_t ld, float* const* mean, float* const* rstd, float eps, int act, int64_t stride_x,
                       int64_t stride_params, int64_t stride_rows, int64_t stride_stats, float* const* WT,
                       int64_t stride_wt);
/* Backward: from dY, the cotangent of the last layer's output, each layer's
 * activation + LayerNorm backward (writes dZ and partial[blocks][2 * 256],
 * the scale | bias gradient sums of each 16-row block, blocks =
 * ppo_mlp_ln_bwd_blocks(M)) and for l > 0 the input cotangent dZ W_l^T read
 * through WT[l] = W_l transposed ([256 out][ldwt], ldwt == 256, as
 * ppo_mlp_ln_fwd_f32 writes it).  The values of ppo_layernorm_act_bwd_f32 and
 * ppo_gemm_f32 (dZ W^T) per layer, up to float32 summation order. */
int ppo_mlp_ln_bwd_blocks(int rows);
int ppo_mlp_ln_bwd_f32(void* stream, int towers, int L, const float* dY, int64_t lddy, int M, const float* const* Z,
                       const float* const* mean, const float* const* rstd, const float* const* gamma,
                       const float* const* beta, const float* const* WT, int64_t ldwt, float* const* dZ, int64_t ld,
                       float* const* partial, int act, int64_t stride_rows, int64_t stride_stats,
                       int64_t stride_params, int64_t stride_wt, int64_t stride_part);

/* ------------------------------------------------ bf16 torso chain
 * The 512-wide Dense -> LayerNorm -> activation layers of a bf16 network
 * (flax Dense / LayerNorm with a bf16 compute dtype, fp32 parameters:
 * boonta/networks/network.py:38-49 as the large-observation workload
 * composes it) after the first layer's split-K contraction, in one launch:
 * layer 0's split sum (split order) + bias, LayerNorm + activation, then for
 * l >= 1 the 512 x 512 contraction of the previous output (bf16 MFMA), bias,
 * LayerNorm + activation.  Writes each layer's Z (the bf16-valued
 * pre-activations), mean, rstd and bf16 output Y16 (row pitch ld), and Y
 * (fp32) where Y != NULL and Y[l] != NULL.  Bit-identical to
 * ppo_splits_bias_act_bf16 + ppo_layernorm_act_fwd_bf16_out16 for layer 0
 * and ppo_gemm_bf16s (bias epilogue, rounded) +
 * ppo_layernorm_act_fwd_bf16_out16 per later layer.  Wp[l] (l >= 1): the
 * layer's kernel as the packed forward operand image that
 * ppo_pack_bf16_operands writes.  With Wh != NULL the launch also computes
 * the Dense head that reads the last layer's output (heads.py:9-45 on a
 * shared torso; nh <= 256 outputs, bias bh, written rounded into head
 * [M][ldh]), bit-identical to ppo_gemm_bf16 with the bias epilogue; Wh is
 * the head kernel's forward operand image from
 * ppo_pack_bf16_operand_padded (n_pad = 32 ceil(nh / 32)).  z16 != 0: Z[l]
 * receives Z as bf16 (uint16 bit patterns; its values are bf16 numbers, so
 * nothing is lost), the form ppo_mlp16_ln_bwd reads with its z16. */
int ppo_mlp16_max_layers(void);
int ppo_mlp16_ln_fwd(void* stream, int L, const float* part, int64_t ldp, int64_t part_stride, int nsplit, int M,
                     const void* const* Wp, const float* const* bias, const float* const* gamma,
                     const float* const* beta, float* const* Z, float* const* Y, void* const* Y16, int64_t ld,
                     float* const* mean, float* const* rstd, float eps, int act, const void* Wh, const float* bh,
                     int nh, float* head, int64_t ldh, int z16);
/* Backward of the same chain from dY, the cotangent of the top layer's
 * output (fp32, row pitch lddy): per layer from the top, the LayerNorm +
 * activation backward (dZ16[l], bf16, row pitch ld, bit-identical to
 * ppo_layernorm_act_bwd_bf16_out16; part[l] [ppo_mlp16_ln_bwd_blocks(M)][2 *
 * 512], the scale | bias gradient sums of each 32-row block) and below the
 * top the input cotangent dZ16[l] W_l^T rounded to bf16 (bit-identical to
 * ppo_gemm_bf16s), read through Wb[l], the packed backward operand image of
 * layer l's kernel.  Replaces, per layer, jax.value_and_grad's LayerNorm,
 * activation and Dense input-cotangent rules (boonta/algorithms/ppo.py:155-157)
 * as the per-layer launches do.  With Whb != NULL dY is not read: the top
 * cotangent is the head's input cotangent dhead W_h^T (dhead [M][lddh], nh
 * columns; Whb the head kernel's backward image from
 * ppo_pack_bf16_operand_padded over nh_pad = 32 or 64 outputs), bit-identical
 * to the bf16 head GEMM's.  z16 != 0: Z[l] holds bf16 (ppo_mlp16_ln_fwd's z16
 * output).  dhead16 (with the head, or NULL): receives the head cotangents
 * rounded to bf16 [M][lddh16] (zero in columns nh .. lddh16 - 1; lddh16 a
 * multiple of 8 between nh and nh_pad), the operand of the head's dW in
 * ppo_gemm_bf16s_dw_group. */
int ppo_mlp16_ln_bwd_blocks(int rows);
int ppo_mlp16_ln_bwd(void* stream, int L, const float* dY, int64_t lddy, int M, const void* const* Wb,
                     const float* const* Z, const float* const* mean, const float* const* rstd,
                     const float* const* gamma, const float* const* beta, void* const* dZ16, int64_t ld,
                     float* const* part, int act, const float* dhead, int64_t lddh, const void* Whb, int nh,
                     int nh_pad, int z16, void* dhead16, int64_t lddh16);
/* Packs L bf16 kernels W[l] ([K][N], row pitch ldw; the bf16 parameter
 * image) into the MFMA operand images of the bf16 chains: fwd[l] for the
 * contraction over K, bwd[l] (W^T) for the input cotangent's contraction over
 * N; K * N bf16 each, 16-byte aligned; NULL entries are skipped.  Layout:
 * 1 KB chunk kb * (ND / 32) + nb holds, for lane l, element i, B[16 kb + 8
 * (l >> 5) + i][32 nb + (l & 31)] of B = W [K][N] (fwd) or W^T [N][K] (bwd).
 * With Wh != NULL the same launch also packs a head kernel Wh [K][nh] (row
 * pitch ldwh) as ppo_pack_bf16_operand_padded does (into fwdh, and bwdh when
 * not NULL). */
int ppo_pack_bf16_operands(void* stream, int L, const void* const* W, int64_t ldw, int K, int N,
                           void* const* fwd, void* const* bwd, const void* Wh, int64_t ldwh, int nh, int nh_pad,
                           void* fwdh, void* bwdh);
/* The operand images of one bf16 kernel [K][N] (row pitch ldw) padded with
 * zeros to n_pad (a multiple of 32 >= N) outputs: a head narrower than the
 * 32-column MFMA blocks.  fwd: the forward operand; bwd (may be NULL): W^T,
 * the operand of the input cotangent's contraction over the n_pad outputs. */
int ppo_pack_bf16_operand_padded(void* stream, const void* W, int64_t ldw, int K, int N, int n_pad, void* fwd,
                                 void* bwd);

/* ------------------------------------------------------- linear scan
 * Replace boonta's linear-recurrence scan and its custom VJP
 * (boonta/networks/kernels/scan.py:13-88: scan / _scan_fwd / _scan_bwd),
 * called by the SSM block (networks/blocks/ssm.py:31-55) behind the MinGRU
 * and other SSM torsos.  a, b, h, cotangent, da, db: [batch, steps, features]
 * row-major; init, dinit: [batch, features]; dtype 0 = float32 storage,
 * 1 = bf16 storage (float32 accumulation in both).
 *   forward:  h_t = a_t h_{t-1} + b_t, h_{-1} = init
 *   backward: db_t = cot_t + a_{t+1} db_{t+1}; da_t = db_t h_{t-1};
 *             dinit = db_0 a_0 */
int ppo_linear_scan_fwd(void* stream, int dtype, const void* a, const void* b, const void* init, void* out,
                        int batch, int steps, int features);
int ppo_linear_scan_bwd(void* stream, int dtype, const void* a, const void* h, const void* init, const void* cot,
                        void* da, void* db, void* dinit, int batch, int steps, int features);
/* The SSM block around the scan (networks/blocks/ssm.py:31-55): where
 * done[n, t] (uint8 [batch, steps]) the step restarts from `reset` ([batch,
 * features], NULL for the zero initial carry of the MinGRU / SSM cells):
 * b' = b + a reset, a' = 0, then the scan from `carry`.  The backward returns
 * the cotangents of a, b and carry through the reset as well. */
int ppo_ssm_scan_fwd(void* stream, int dtype, const void* a, const void* b, const uint8_t* done, const void* reset,
                     const void* carry, void* out, int batch, int steps, int features);
int ppo_ssm_scan_bwd(void* stream, int dtype, const void* a, const void* h, const uint8_t* done, const void* reset,
                     const void* carry, const void* cot, void* da, void* db, void* dcarry, int batch, int steps,
                     int features);

/* ------------------------------------------------------------------ GEMM
 * Dense layers of the torso and heads (flax.linen.Dense as composed in
 * hangar/recipes/*.py; forward at boonta/networks/network.py:38-49, backward
 * of jax.value_and_grad at boonta/algorithms/ppo.py:155-157), fp32 MFMA.
 * C[m][n] (+ split * c_split_stride) = epilogue(sum_k A(m,k) B(k,n))
 *   a_layout 0: A[m*lda + k]   1: A[k*lda + m]
 *   b_layout 0: B[k*ldb + n]   1: B[n*ldb + k]
 *   rows: gather of A's rows (layout 0 over m, layout 1 over k), or NULL
 *   epi 0: store; 1: + bias[n], activation `act` (pre-activation to `pre`);
 *       2: multiply by act'(aux) (aux: activation output for relu/tanh,
 *       input for silu)
 *   splits > 1: split of the reduction; partial s at C + s * c_split_stride
 *   bias_grad (a_layout 1, b_layout 0): [splits][N] column sums of B
 *   tile: -1 automatic (64x64); 0 128x128, 1 128x64, 2 64x128, 3 64x64
 *   (operands copied straight into LDS, 32 reduction steps per stage); 4-7
 *   the same tiles staged through registers; 8 128x256, 9 256x128 (8 waves,
 *   copied straight into LDS). */
int ppo_gemm_f32(void* stream, int a_layout, int b_layout, const float* A, int64_t lda, const int32_t* rows,
                 const float* B, int64_t ldb, float* C, int64_t ldc, int M, int N, int K, int splits,
                 int64_t c_split_stride, int epi, const float* bias, int act, float* pre, const float* aux,
                 int64_t ldaux, float* bias_grad, int tile);
/* ppo_gemm_f32 for `towers` (<= 8) contractions of one shape in one grid
 * (the actor and critic towers' forward, dW and input-cotangent products):
 * contraction t reads A, B, bias and aux and writes C, pre and bias_grad at
 * t times the given element strides after contraction 0's (a stride of 0
 * shares the operand; the row gather `rows` is shared).  Bit-identical to
 * one ppo_gemm_f32 per tower. */
int ppo_gemm_f32_towers(void* stream, int towers, int a_layout, int b_layout, const float* A, int64_t lda,
                        const int32_t* rows, const float* B, int64_t ldb, float* C, int64_t ldc, int M, int N, int K,
                        int splits, int64_t c_split_stride, int epi, const float* bias, int act, float* pre,
                        const float* aux, int64_t ldaux, float* bias_grad, int tile, int64_t stride_a,
                        int64_t stride_b, int64_t stride_c, int64_t stride_bias, int64_t stride_pre,
                        int64_t stride_aux, int64_t stride_bias_grad);

/* bf16 compute (flax Dense with dtype=bfloat16, param_dtype=float32; the
 * mixed precision of boonta/networks/README.md:73-77): the same contraction
 * and layouts as ppo_gemm_f32 on v_mfma_f32_32x32x16_bf16 with fp32
 * accumulation.  Operands stay fp32 in memory and are rounded to bf16 (round
 * to nearest even) as they are read: the casts of the input, the kernel and
 * any fp32 cotangent.  round_out != 0 rounds the result to bf16 (and with
 * epi 1 adds the bf16-rounded bias and rounds again, then the activation);
 * round_out = 0 keeps fp32 (dW partials, rounded after their sum by
 * ppo_grad_reduce). */
int ppo_gemm_bf16(void* stream, int a_layout, int b_layout, const float* A, int64_t lda, const int32_t* rows,
                  const float* B, int64_t ldb, float* C, int64_t ldc, int M, int N, int K, int splits,
                  int64_t c_split_stride, int epi, const float* bias, int act, int round_out, const float* aux,
                  int64_t ldaux, float* bias_grad, int tile);
/* x[i] <- bf16(x[i]) in place (the fp32 value of the nearest-even bf16). */
int ppo_round_bf16(void* stream, float* x, int64_t n);
/* The same contraction for long reductions (the first layer of a bf16 network
 * over thousands of observation features), pipelined for bf16 MFMA rates
 * (256 x 128 tiles, 8 waves, BK 64, loads two stages ahead).  a_bf16 / b_bf16:
 * the operand is stored as bf16 bit patterns (the observation copy, the bf16
 * image of the parameters) instead of fp32.  Rows must be 16-byte aligned; a
 * bf16 operand's row pitch is at least its contiguous extent rounded up to 8.
 * With both operands stored as bf16, stages are copied straight from global
 * memory into LDS (no register staging), three stages in flight.
 * tile: -1 picks; 0: 256 x 128 (8 waves), 1: 128 x 128 (4 waves), 2: 256 x 256
 * (8 waves, two stages; both operands bf16, otherwise tile 0). */
int ppo_gemm_bf16s(void* stream, int a_layout, int b_layout, int a_bf16, int b_bf16, const void* A, int64_t lda,
                   const int32_t* rows, const void* B, int64_t ldb, float* C, int64_t ldc, int M, int N, int K,
                   int splits, int64_t c_split_stride, int epi, const float* bias, int act, int round_out,
                   const float* aux, int64_t ldaux, float* bias_grad, int tile);
/* The weight gradients of up to 8 fp32 Dense layers in one launch (a
 * backward pass's dW GEMMs, so that a layer with few tiles runs beside one
 * with many instead of after it): problem i (host arrays, one entry per
 * problem; rows and bias_grad may be NULL, or hold NULL entries) is exactly
 * ppo_gemm_f32(stream, 1, 0, A[i], lda[i], rows[i], B[i], ldb[i], C[i], ldc[i],
 * M[i], N[i], K[i], splits[i], c_split_stride[i], 0, NULL, 0, NULL, NULL, 0,
 * bias_grad[i], 3), same bits, when every operand row is 16-byte vectorisable
 * (lda, ldb, M[i], N[i] multiples of 4; 16-byte aligned A, B).  A gathered
 * problem's split holds at most 2048 rows.  Part of the backward pass of
 * jax.value_and_grad at boonta/algorithms/ppo.py:155-157 (the Dense kernel and
 * bias cotangents). */
int ppo_gemm_f32_dw_group(void* stream, int count, const float* const* A, const int64_t* lda,
                          const int32_t* const* rows, const float* const* B, const int64_t* ldb, float* const* C,
                          const int64_t* ldc, const int* M, const int* N, const int* K, const int* splits,
                          const int64_t* c_split_stride, float* const* bias_grad);
/* Output tiles (64 x 64) of a weight-gradient group of count problems of
 * M[i] x N[i] (all positive): the arrival counters and squared-norm slots of
 * ppo_gemm_f32_dw_group_final, problem after problem; -1 on a bad shape. */
int ppo_gemm_f32_dw_final_slots(int count, const int* M, const int* N);
/* ppo_gemm_f32_dw_group with the gradient assembly of its problems in the
 * same launch (the ppo_grad_reduce launch that would follow it is not
 * needed): the split partials C[i] / bias_grad[i] are written as before, and
 * the last split of each 64 x 64 output tile to finish sums them in
 * ppo_grad_reduce's fixed order into the final gradient G[i] (rows below
 * g_rows[i] <= M[i], row pitch ldg[i]; a zero-padded input's extra rows are
 * dropped) and the bias gradient Gb[i] (skipped when Gb or Gb[i] is NULL),
 * and writes the tile's squared-norm partial to sumsq[slot] (slots and
 * counters numbered tile by tile, problem after problem, as
 * ppo_gemm_f32_dw_final_slots counts them).  The gradient segments of the
 * ppo_grad_reduce tables segs / chunks (their chunk slots numbered after the
 * tiles') are reduced by workgroups of the same launch.  counters: nine
 * zeroed unsigneds per tile (the last eight per tile for the two-level sums),
 * left zeroed; calls sharing counters must not overlap.  The gradients are
 * the same bits as ppo_gemm_f32_dw_group followed by ppo_grad_reduce (the
 * norm partials are grouped by tile instead of by chunk).  splits[i] in
 * {1, 2, 3, 4, 6, 8, 12, 16} (one level) or {32, 64} (the last of each group
 * of eight splits sums it, the last group the group sums); a gathered split
 * holds at most 512 rows; all problems non-empty.  Replaces the weight-gradient GEMMs and gradient
 * assembly of jax.value_and_grad at boonta/algorithms/ppo.py:155-157. */
int ppo_gemm_f32_dw_group_final(void* stream, int count, const float* const* A, const int64_t* lda,
                                const int32_t* const* rows, const float* const* B, const int64_t* ldb,
                                float* const* C, const int64_t* ldc, const int* M, const int* N, const int* K,
                                const int* splits, const int64_t* c_split_stride, float* const* bias_grad,
                                float* const* G, const int64_t* ldg, const int* g_rows, float* const* Gb,
                                unsigned* counters, double* sumsq, const void* segs, const void* chunks, int nchunks,
                                int nfew, int nwide);
/* The weight gradients of up to 8 bf16 Dense layers in one launch (one
 * backward pass's dW GEMMs, so that a layer with few tiles runs beside one with
 * many instead of after it): problem i (host arrays, one entry per problem;
 * rows and bias_grad may be NULL, or hold NULL entries) is exactly
 * ppo_gemm_bf16s(stream, 1, 0, 1, 1, A[i], lda[i], rows[i], B[i], ldb[i], C[i],
 * ldc[i], M[i], N[i], K[i], splits[i], c_split_stride[i], 0, NULL, 0, 0, NULL,
 * 0, bias_grad[i], 2), same bits.  A gathered problem's split holds at most
 * 4096 rows.  Part of the backward pass of jax.value_and_grad at
 * boonta/algorithms/ppo.py:155-157 (the Dense kernel and bias cotangents). */
int ppo_gemm_bf16s_dw_group(void* stream, int count, const void* const* A, const int64_t* lda,
                            const int32_t* const* rows, const void* const* B, const int64_t* ldb, float* const* C,
                            const int64_t* ldc, const int* M, const int* N, const int* K, const int* splits,
                            const int64_t* c_split_stride, float* const* bias_grad);
/* Row-pitched float32 copy padded with zeros: y[r][c] = x[r][c] for c < cols,
 * 0 for cols <= c < ldy (ldy a multiple of 4, y 16-byte aligned).  The
 * per-update copy of observation rows whose width is not a multiple of four
 * (obs [16, 4096, 87] of the Gaussian workload), which lets the first layer's
 * weight gradient (ppo.py:148-151 gather, then the Dense of
 * networks/network.py:18-49 under jax.grad) run on the copy-fed GEMM over the
 * padded width; the pad columns' gradient rows are never read. */
int ppo_pad_rows_f32(void* stream, const float* x, int64_t ldx, float* y, int64_t ldy, int rows, int cols);
/* y[i] = bf16(x[i]) as 16-bit patterns (the bf16 parameter image); 16-byte aligned. */
int ppo_cast_bf16(void* stream, const float* x, void* y, int64_t n);
/* Row-pitched bf16 copy (the per-update observation copy): y[r][c] = bf16(x[r][c])
 * for c < cols, 0 for cols <= c < ldy; ldy a multiple of 8, ldx of 4, both
 * buffers 16-byte aligned. */
int ppo_cast_bf16_2d(void* stream, const float* x, int64_t ldx, void* y, int64_t ldy, int rows, int cols);
/* out[r][j] = act(bf16(bf16(sum_s partials[s][r][j]) + bf16(bias[j]))), each step
 * rounded to bf16 (flax's Dense in bf16 after a split-K contraction; bias may
 * be NULL, act 0 = none).  Partials are added in split order. */
int ppo_splits_bias_act_bf16(void* stream, const float* partials, int64_t ldp, int64_t split_stride, int nsplit,
                             const float* bias, int act, float* out, int64_t ldc, int rows, int cols);

/* ------------------------------------------------------ LayerNorm / act
 * flax.linen.LayerNorm (epsilon, fast variance, scale and bias) followed by
 * an activation, as the Dense -> LayerNorm -> act blocks of the configs.
 * Forward stores per-row mean/rstd for the backward. */
int ppo_layernorm_act_fwd_f32(void* stream, const float* z, int64_t ldz, const float* gamma, const float* beta,
                              float* y, int64_t ldy, float* mean, float* rstd, int rows, int F, float eps,
                              int act);
int ppo_layernorm_bwd_blocks(int rows);
/* dy: cotangent of the activation output; writes dz and partial[blocks][2F]
 * (scale | bias gradient sums per block). */
int ppo_layernorm_act_bwd_f32(void* stream, const float* dy, int64_t lddy, const float* z, int64_t ldz,
                              const float* mean, const float* rstd, const float* gamma, const float* beta,
                              float* dz, int64_t lddz, float* partial, int rows, int F, int act);
/* The same backward for `towers` (<= 8) layers of one shape in one grid:
 * tower t's dy / z / dz rows, mean / rstd, gamma / beta and partials sit
 * t times the given element strides after tower 0's.  Bit-identical to one
 * ppo_layernorm_act_bwd_f32 per tower. */
int ppo_layernorm_act_bwd_f32_towers(void* stream, int towers, const float* dy, int64_t lddy, const float* z,
                                     int64_t ldz, const float* mean, const float* rstd, const float* gamma,
                                     const float* beta, float* dz, int64_t lddz, float* partial, int rows, int F,
                                     int act, int64_t stride_rows, int64_t stride_stats, int64_t stride_params,
                                     int64_t stride_part);
/* bf16 compute: flax's LayerNorm with dtype=bfloat16 computes statistics and
 * the normalisation in fp32 and casts the result to bf16 before the
 * activation; the backward rounds the input cotangent to bf16. */
int ppo_layernorm_act_fwd_bf16(void* stream, const float* z, int64_t ldz, const float* gamma, const float* beta,
                               float* y, int64_t ldy, float* mean, float* rstd, int rows, int F, float eps,
                               int act);
/* ppo_layernorm_act_fwd_bf16 that also stores y as bf16 bit patterns (y16,
 * row pitch ldy16 elements): the operand of the next bf16 contraction.  y
 * may be NULL when only the bf16 copy is read afterwards. */
int ppo_layernorm_act_fwd_bf16_out16(void* stream, const float* z, int64_t ldz, const float* gamma, const float* beta,
                                     float* y, int64_t ldy, void* y16, int64_t ldy16, float* mean, float* rstd,
                                     int rows, int F, float eps, int act);
int ppo_layernorm_act_bwd_bf16(void* stream, const float* dy, int64_t lddy, const float* z, int64_t ldz,
                               const float* mean, const float* rstd, const float* gamma, const float* beta,
                               float* dz, int64_t lddz, float* partial, int rows, int F, int act);
/* ppo_layernorm_act_bwd_bf16 with dz stored as bf16 bit patterns (row pitch
 * lddz16 elements): the operand of a bf16 dW contraction. */
int ppo_layernorm_act_bwd_bf16_out16(void* stream, const float* dy, int64_t lddy, const float* z, int64_t ldz,
                                     const float* mean, const float* rstd, const float* gamma, const float* beta,
                                     void* dz16, int64_t lddz16, float* partial, int rows, int F, int act);
int ppo_act_fwd_f32(void* stream, const float* x, int64_t ldx, float* y, int64_t ldy, int rows, int F, int act);
int ppo_act_bwd_f32(void* stream, const float* dy, int64_t lddy, const float* aux, int64_t ldaux, float* dx,
                    int64_t lddx, int rows, int F, int act);

/* ------------------------------------------------------------------ loss
 * Replaces loss_fn of boonta/algorithms/ppo.py:77-146 (recurrent_ppo.py:101-184)
 * with distrax Categorical / MultivariateNormalDiag of
 * boonta/networks/distributions.py:8-57, and its cotangent w.r.t. the head
 * outputs.  head: logits [rows, A] or Gaussian mean [rows, A] (+ raw scale at
 * column A + j when scale_param is NULL); value at value[r * ldv].  Per-sample
 * inputs are indexed through idx (minibatch row -> sample).  Writes dhead,
 * dvalue (same layouts), stats_partial[blocks][ppo_loss_stat_count()] and,
 * for a state-independent scale, dscale_partial[blocks][A]. */
int ppo_loss_blocks(int rows);
int ppo_loss_stat_count(void);
int ppo_loss_f32(void* stream, int dist, int rows, const int32_t* idx, const float* head, int64_t ldh,
                 const float* value, int64_t ldv, int A, const float* scale_param, const int32_t* action_i,
                 const float* action_f, const float* old_logp, const float* old_value, const float* adv,
                 const float* ret, float* dhead, float* dvalue, float* dscale_partial, double* stats_partial,
                 float clip_eps, int clip_value_loss, float ent_coef, float vf_coef, float temperature);
/* The logged scalars of ppo.py:170-179 in order, then the total loss: out9[9]. */
int ppo_loss_finalize(void* stream, const double* stats_partial, int nblocks, int rows, float ent_coef,
                      float vf_coef, float* out9);
/* The same for `steps` optimizer steps at once, off the minibatch chain:
 * stats_partial [steps][nblocks][11] -> out [steps][9] (one launch per update
 * instead of one per step; the logs of ppo.py:170-180 are not an input of any
 * later step). */
int ppo_loss_finalize_steps(void* stream, const double* stats_partial, int nblocks, int rows, int steps,
                            float ent_coef, float vf_coef, float* out);

/* Fused heads + loss + head backward: one wavefront per sample row reads the
 * torso output once.  Group a is the actor head, or both heads packed into one
 * [F, ldwa] matrix with the value in column na - 1 when hc is NULL; group c is
 * the critic head of separate towers.  Writes the cotangent of each head input
 * (times act'(aux) when act != NONE), per-block head weight / bias gradient
 * partials [blocks][F][ld] / [blocks][ld] (blocks = ppo_head_loss_blocks(rows)),
 * statistics and Gaussian scale partials as ppo_loss_f32 does.  F <= 512,
 * na <= 16.  sample_stride: elements between consecutive samples of
 * old_logp, old_value, adv, ret and action_i (1: separate columns; 8: the
 * records of ppo_pack_samples, old_logp = rec, old_value = rec + 1, adv =
 * rec + 2, ret = rec + 3, action_i = rec + 4, whose four scalars a row then
 * reads in one 16-byte load). */
int ppo_head_loss_blocks(int rows);
int ppo_head_loss_max_outputs(void);
int ppo_head_loss_max_features(void);
int ppo_head_loss_f32(void* stream, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha,
                      const float* wa, int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc,
                      const float* wc, int64_t ldwc, const float* bc, int F, int A, const float* scale_param,
                      const int32_t* action_i, const float* action_f, const float* old_logp,
                      const float* old_value, const float* adv, const float* ret, int act_a, const float* aux_a,
                      int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
                      int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a,
                      float* wpart_c, float* bpart_c, float* dscale_partial, double* stats_partial,
                      float clip_eps, int clip_value_loss, float ent_coef, float vf_coef, float temperature,
                      int64_t sample_stride);
/* The per-sample rollout inputs of the fused loss (the gathers of
 * boonta/algorithms/ppo.py:148-151 for log_prob, value, advantages, returns
 * and categorical actions) as one 32-byte record per sample, written once per
 * update after the advantages are final: rec[8 s .. 8 s + 7] = {old_logp,
 * old_value, adv, ret, action_i bits (0 when action_i is NULL), 0, 0, 0}.
 * rec 16-byte aligned. */
int ppo_pack_samples(void* stream, int64_t n, const float* old_logp, const float* old_value, const float* adv,
                     const float* ret, const int32_t* action_i, float* rec);
/* The forward chain of an actor / critic pair of towers followed, in the same
 * launch, by their fused heads + PPO loss on the chains' last outputs: what
 * ppo_mlp_ln_fwd_f32(stream, <its arguments>) then ppo_head_loss_f32(stream,
 * <the remaining arguments>) compute, bit for bit (each tower's workgroups
 * run that tower's half of the loss on the tile they hold in LDS).  Requires
 * towers = 2, separate heads (hc non-NULL) over F = 256 features with no
 * activation derivative (act_a = act_c = 0), ha = Y[L - 1], hc = ha +
 * stride_rows, ldha = ldhc = ld, rows = M, and M within the head loss's
 * 16-row-block range (ppo_head_loss_blocks(M) = ceil(M / 16)).  Replaces the
 * torso forward of boonta/networks/network.py:38-49 and loss_fn of
 * boonta/algorithms/ppo.py:77-146 with its head backward, for flax's
 * ActorCritic with separate LayerNorm torsos. */
int ppo_mlp_ln_fwd_head_loss_f32(
    void* stream, int towers, int L, const float* X, int64_t ldx, const int32_t* rows_idx, int M, int K0,
    const float* const* W, int64_t ldw0, int64_t ldw, const float* const* bias, const float* const* gamma,
    const float* const* beta, float* const* Z, float* const* Y, int64_t ld, float* const* mean, float* const* rstd,
    float eps, int act, int64_t stride_x, int64_t stride_params, int64_t stride_rows, int64_t stride_stats,
    float* const* WT, int64_t stride_wt, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha,
    const float* wa, int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc,
    int64_t ldwc, const float* bc, int F, int A, const float* scale_param, const int32_t* action_i,
    const float* action_f, const float* old_logp, const float* old_value, const float* adv, const float* ret,
    int act_a, const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature, int64_t sample_stride);
/* ppo_mlp_ln_fwd_head_loss_f32 followed by ppo_mlp_ln_bwd_f32 from the heads'
 * input cotangents, in one launch, bit for bit (each workgroup runs the
 * backward of its own 16 rows after their forward and loss: every row's loss
 * cotangent depends only on that row).  The chain and head arguments are
 * those of ppo_mlp_ln_fwd_head_loss_f32 except WT / stride_wt: the transposed
 * kernels of layers 1..L-1 that the backward reads, written before this
 * launch (e.g. by ppo_adam_clip_wt_f32); this launch writes none.  The
 * backward reads dY = dha (tower 1: dhc = dha + stride_rows, lddhc = lddha)
 * and writes dZ[l] (row pitch ld) and the LayerNorm parameter partials
 * partial[l] (tower stride stride_part) as ppo_mlp_ln_bwd_f32 does.  Replaces
 * the same reference code as those two entry points (the torso forward of
 * boonta/networks/network.py:38-49, loss_fn of boonta/algorithms/ppo.py:77-146
 * and its backward under jax.value_and_grad, ppo.py:155-157). */
int ppo_mlp_ln_fwd_head_loss_bwd_f32(
    void* stream, int towers, int L, const float* X, int64_t ldx, const int32_t* rows_idx, int M, int K0,
    const float* const* W, int64_t ldw0, int64_t ldw, const float* const* bias, const float* const* gamma,
    const float* const* beta, float* const* Z, float* const* Y, int64_t ld, float* const* mean, float* const* rstd,
    float eps, int act, int64_t stride_x, int64_t stride_params, int64_t stride_rows, int64_t stride_stats,
    float* const* WT, int64_t stride_wt, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha,
    const float* wa, int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc, const float* wc,
    int64_t ldwc, const float* bc, int F, int A, const float* scale_param, const int32_t* action_i,
    const float* action_f, const float* old_logp, const float* old_value, const float* adv, const float* ret,
    int act_a, const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c, const float* aux_c,
    int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a, float* bpart_a, float* wpart_c, float* bpart_c,
    float* dscale_partial, double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
    float vf_coef, float temperature, int64_t sample_stride, float* const* dZ, float* const* partial,
    int64_t stride_part);
/* ppo_head_loss_f32 that also keeps each row's ratio exp(logp - old_logp),
 * env-major: ratio_out[(s % envs) * steps + s / envs] for the row's sample
 * s = idx[row] = t * envs + env (the new ratio RecurrentPuPO scatters back
 * with stop_gradient, recurrent_pupo.py:123,297). */
int ppo_head_loss_ratio_f32(void* stream, int dist, int rows, const int32_t* idx, const float* ha, int64_t ldha,
                            const float* wa, int64_t ldwa, const float* ba, int na, const float* hc, int64_t ldhc,
                            const float* wc, int64_t ldwc, const float* bc, int F, int A, const float* scale_param,
                            const int32_t* action_i, const float* action_f, const float* old_logp,
                            const float* old_value, const float* adv, const float* ret, int act_a,
                            const float* aux_a, int64_t ldaux_a, float* dha, int64_t lddha, int act_c,
                            const float* aux_c, int64_t ldaux_c, float* dhc, int64_t lddhc, float* wpart_a,
                            float* bpart_a, float* wpart_c, float* bpart_c, float* dscale_partial,
                            double* stats_partial, float clip_eps, int clip_value_loss, float ent_coef,
                            float vf_coef, float temperature, float* ratio_out, int envs, int steps,
                            int64_t sample_stride);

/* ------------------------------------------------------------------- GRU
 * One time step of flax.linen.GRUCell inside boonta's RNN block
 * (boonta/networks/blocks/rnn.py:34-54, reset_carry :11-16), forward and
 * backward, for a time-major batch of Bm sequences; replaces the nn.scan
 * forward and its BPTT under jax.value_and_grad in
 * boonta/algorithms/recurrent_ppo.py:101-184.  H must be a multiple of 64.
 *   xi     [Bm, 3H] input projections x Wi + bi, columns (n | r | z)
 *   wh     [H, 3H]  recurrent kernels, columns (r | z | n); bhn [H]
 *   gates  [Bm, 4H] saved (n | r | z | hn); dgate [Bm, 4H] (dan | dar | daz | dhn)
 * Forward: h_prev row b is hprev[(hprev_rows ? hprev_rows[b] : b) * ldh]; it
 * is replaced by zeros where terminated[i] | truncated[i], i = flag_rows ?
 * flag_rows[b] : b (flags may be NULL: no reset).  Writes h_out, and when
 * non-NULL hp_out (the reset previous carry) and gates.
 * Backward at step t (dg = dgate_t + H, or NULL for the first call at the
 * last step): dh_s = dout_s + (reset_t ? 0 : dg Wh^T + dh_t * z_t), then the
 * gate cotangents of step s = t - 1 into dgate_s. */
int ppo_gru_fwd_step_f32(void* stream, const float* xi, int64_t ldxi, const float* hprev, int64_t ldh,
                         const int32_t* hprev_rows, const uint8_t* terminated, const uint8_t* truncated,
                         const int32_t* flag_rows, const float* wh, int64_t ldwh, const float* bhn, float* h_out,
                         int64_t ldo, float* hp_out, int64_t ldhp, float* gates, int64_t ldg, int Bm, int H);
int ppo_gru_bwd_step_f32(void* stream, const float* dg, int64_t lddg, const float* wh, int64_t ldwh,
                         const float* dh_t, int64_t lddht, const float* z_t, int64_t ldz, const uint8_t* terminated,
                         const uint8_t* truncated, const int32_t* flag_rows, const float* dout, int64_t lddo,
                         const float* gates_s, int64_t ldg, const float* hp_s, int64_t ldhp, float* dh_s,
                         int64_t lddhs, float* dgate_s, int64_t lddgs, int Bm, int H);
/* The whole recurrence of a sequence minibatch in one launch per direction
 * (the loop of boonta/networks/blocks/rnn.py:34-54 over T steps, and its
 * backward through time): workgroup (x, y) keeps sequences 16x..16x+15 and
 * units 16y..16y+15 for every step with its slice of Wh in LDS; the
 * workgroups of a sequence block hand each step to the next through
 * `exchange` (ppo_gru_seq_exchange_bytes(Bm, H) bytes, 16-byte aligned,
 * zeroed by the call), as {value, step tag} pairs that a consumer polls until
 * the tag is the step's.  Each wait polls at most spin_limit times (0: none,
 * to exercise the error path);
 * a wait that gives up sets *error to 1 and its workgroup ends, so the launch
 * always completes.  Needs ceil(Bm / 16) * H / 16 <=
 * ppo_gru_seq_max_workgroups() (all workgroups resident) and H <= 256.
 * The values are those of T ppo_gru_fwd_step_f32 / ppo_gru_bwd_step_f32
 * launches, bit for bit.  Step t's operands sit at the base pointers plus t
 * times the *_step strides (elements; flag_rows + t * flag_step). */
int ppo_gru_seq_max_workgroups(void);
int64_t ppo_gru_seq_exchange_bytes(int Bm, int H);
int ppo_gru_fwd_seq_f32(void* stream, const float* xi, int64_t ldxi, int64_t xi_step, const float* h0, int64_t ldh0,
                        const int32_t* h0_rows, const uint8_t* terminated, const uint8_t* truncated,
                        const int32_t* flag_rows, int64_t flag_step, const float* wh, int64_t ldwh, const float* bhn,
                        float* h_out, int64_t ldo, int64_t h_step, float* hp_out, int64_t ldhp, int64_t hp_step,
                        float* gates, int64_t ldg, int64_t g_step, int Bm, int H, int T, void* exchange,
                        int* error, int spin_limit);
int ppo_gru_bwd_seq_f32(void* stream, const float* wh, int64_t ldwh, const uint8_t* terminated,
                        const uint8_t* truncated, const int32_t* flag_rows, int64_t flag_step, const float* dout,
                        int64_t lddo, int64_t dout_step, const float* gates, int64_t ldg, int64_t g_step,
                        const float* hp, int64_t ldhp, int64_t hp_step, float* dh, int64_t lddh, int64_t dh_step,
                        float* dgate, int64_t lddg, int64_t dg_step, int Bm, int H, int T, void* exchange,
                        int* error, int spin_limit);
/* ppo_gru_fwd_seq_f32 with the input projections made in the same launch
 * (the x Wi + bi of the flax GRUCell, boonta/networks/blocks/rnn.py:34-54,
 * for every step instead of one GEMM launch before the recurrence): xi = e
 * Wi + bi for the GRU input e of row t Bm + b at e + t e_step + b lde, wi
 * [I][3H] with row pitch ldwi and bi [3H] in columns [n|r|z].  Each step's
 * products are summed in a fixed order of their own, so the results equal
 * ppo_gru_fwd_seq_f32 on a GEMM's xi to rounding, not bit for bit.  H = I =
 * 256; e rows 16-byte aligned.  ring_is_zero: the exchange ring is already
 * zero, so the launch does not zero it first; clear_ring / clear_bytes (or
 * NULL / 0): a second ring (the backward's) that the launch leaves zero as
 * its workgroups finish — with one ring per direction, each sequence launch
 * leaves the other's ring ready and neither needs a zeroing launch (zero
 * both once, and again after a launch that set the error word). */
int ppo_gru_fwd_seq_xw_f32(void* stream, const float* h0, int64_t ldh0, const int32_t* h0_rows,
                           const uint8_t* terminated, const uint8_t* truncated, const int32_t* flag_rows,
                           int64_t flag_step, const float* wh, int64_t ldwh, const float* bhn, float* h_out,
                           int64_t ldo, int64_t h_step, float* hp_out, int64_t ldhp, int64_t hp_step, float* gates,
                           int64_t ldg, int64_t g_step, int Bm, int H, int T, void* exchange, int* error,
                           int spin_limit, const float* e, int64_t lde, int64_t e_step, int I, const float* wi,
                           int64_t ldwi, const float* bi, int ring_is_zero, void* clear_ring, int64_t clear_bytes);
/* ppo_gru_bwd_seq_f32 that also leaves the weight gradients of the GRU's
 * input and recurrent Dense kernels and their biases (the flax GRUCell of
 * boonta/networks/blocks/rnn.py:34-54 under jax.value_and_grad,
 * recurrent_ppo.py:213-215), multiplied while the launch waits for its
 * exchange loads, as P = ppo_gru_seq_dw_parts(Bm) partials (one per block of
 * 16 sequences, over its rows and every step; the gradient reduce sums them):
 *   whpart [P][H][3H] = hp^T dgate[:, H:4H]     whbpart [P][3H]: column sums of dgate[:, H:4H]
 *   wipart [P][I][3H] = e^T dgate[:, 0:3H]      wibpart [P][3H]: column sums of dgate[:, 0:3H]
 * where e is the GRU input of row t Bm + b at e + t e_step + b lde.  dh and
 * dgate are those of ppo_gru_bwd_seq_f32, bit for bit.  H = I = 256; hp and
 * e rows 16-byte aligned.  ring_is_zero, clear_ring, clear_bytes: as for
 * ppo_gru_fwd_seq_xw_f32 (here clear_ring is the forward's ring). */
int ppo_gru_seq_dw_parts(int Bm);
int ppo_gru_bwd_seq_dw_f32(void* stream, const float* wh, int64_t ldwh, const uint8_t* terminated,
                           const uint8_t* truncated, const int32_t* flag_rows, int64_t flag_step, const float* dout,
                           int64_t lddo, int64_t dout_step, const float* gates, int64_t ldg, int64_t g_step,
                           const float* hp, int64_t ldhp, int64_t hp_step, float* dh, int64_t lddh, int64_t dh_step,
                           float* dgate, int64_t lddg, int64_t dg_step, int Bm, int H, int T, void* exchange,
                           int* error, int spin_limit, const float* e, int64_t lde, int64_t e_step, int I,
                           float* whpart, float* whbpart, float* wipart, float* wibpart, int ring_is_zero,
                           void* clear_ring, int64_t clear_bytes);
/* Sample rows of S env-major sequence minibatches (recurrent_ppo.py:217-223):
 * out[s * T * Bm + t * Bm + b] = t * N + envs[s * Bm + b]. */
int ppo_sequence_rows(void* stream, const int32_t* envs, int S, int T, int N, int Bm, int32_t* out);

/* ------------------------------------------------------------- optimizer
 * Replaces optax.chain(optax.clip_by_global_norm(max_norm), optax.adam(lr))
 * .update + optax.apply_updates at boonta/algorithms/ppo.py:182-191 (chain
 * built at hangar/recipes/ppo_cartpole.py:44-47), on flat fp32 buffers.
 * ppo_grad_reduce sums the partials of every gradient leaf into the flat
 * gradient (device tables of segments and chunks) and leaves one sum of
 * squares per chunk; ppo_adam_clip_f32 folds them into the global norm.
 * A segment is {float* dst; const float* src; int64 count; int64
 * part_stride; int32 nparts; int32 flags} (flags bit 0: round the summed
 * gradient to bf16, for parameters a bf16-compute layer casts); a chunk is
 * {int32 segment; int32 slot; int64 start} covering
 * ppo_grad_reduce_chunk_elems() elements, whose sum of squares lands in
 * sumsq[slot].  The first nfew chunks (0 <= nfew <= nchunks) must belong to
 * segments with at most ppo_grad_reduce_few_parts() partials: they take a
 * path with more loads in flight that gives the same bits.  The last nwide
 * chunks (nfew + nwide <= nchunks) cover ppo_grad_reduce_wide_chunk_elems()
 * elements each, of segments with more than ppo_grad_reduce_wide_parts()
 * partials: sixteen partial ranges summed side by side, then added in range
 * order (a fixed order of its own).
 * The optax count is count_base[0] + step_offset + 1 (device int32). */
int ppo_grad_reduce_segment_bytes(void);
int ppo_grad_reduce_chunk_bytes(void);
int ppo_grad_reduce_chunk_elems(void);
int ppo_grad_reduce_few_parts(void);
int ppo_grad_reduce_wide_parts(void);
int ppo_grad_reduce_wide_chunk_elems(void);
int ppo_grad_reduce(void* stream, const void* segs, const void* chunks, int nchunks, int nfew, int nwide,
                    double* sumsq);
/* params_bf16 (may be NULL): receives the bf16 image of the updated parameters.
 * abort_word (may be NULL): a device int32; when it is nonzero at the time the
 * launch runs (e.g. the error word of a GRU sequence launch of this update
 * whose bounded wait gave up), the step writes nothing, so parameters and
 * moments keep their values. */
int ppo_adam_clip_f32(void* stream, float* params, const float* grads, float* mu, float* nu, void* params_bf16,
                      int64_t n, const double* sumsq, int nsumsq, double max_norm, double lr, double b1,
                      double b2, double eps, const int* count_base, int step_offset, const int* abort_word);
/* ppo_adam_clip_f32 that also writes the transposed image of ntr (at most 8)
 * 256 x 256 row-major kernels inside the parameters: kernel r starts at
 * element tr_off[r] (a multiple of 4; kernels disjoint) and its updated
 * values go to tr_dst[r] as [256 out][256 in] (16-byte aligned), the operand
 * ppo_mlp_ln_fwd_head_loss_bwd_f32's backward reads.  Parameters, moments and
 * bf16 image are the same bits as ppo_adam_clip_f32's; with an abort word set
 * nothing is written.  Replaces the same optax update as ppo_adam_clip_f32
 * (boonta/algorithms/ppo.py:182-191). */
int ppo_adam_clip_wt_f32(void* stream, float* params, const float* grads, float* mu, float* nu, void* params_bf16,
                         int64_t n, const double* sumsq, int nsumsq, double max_norm, double lr, double b1,
                         double b2, double eps, const int* count_base, int step_offset, const int* abort_word,
                         int ntr, const int64_t* tr_off, float* const* tr_dst);
/* total[0] = sum of sumsq[0..n) in a fixed order (one block of 1024 threads):
 * the squared global norm, handed to ppo_adam_clip_f32 as one partial. */
int ppo_sumsq_total(void* stream, const double* sumsq, int n, double* total);
/* count_base[0] += steps, unless abort_word (may be NULL) is nonzero. */
int ppo_count_advance(void* stream, int* count_base, int steps, const int* abort_word);

#ifdef __cplusplus
}
#endif

#endif /* PPO_HIP_H_ */
