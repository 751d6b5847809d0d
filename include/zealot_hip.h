/* zealot_hip.h — C ABI of libzealot_hip.so, the MI355X (gfx950) PPO learning
 * hot path for zealot-rl.
 *
 * Plain C: opaque handles, raw device pointers, sizes and status codes; no
 * exceptions cross this boundary. Every compute entry point is enqueued on
 * the context's single HIP stream and is asynchronous unless it says
 * otherwise; ordering between calls is stream (issue) order, as with the
 * cuTile adapter it replaces (src/biped/cutile_gemm.rs:15-27).
 *
 * Device buffers passed in are BORROWED: the library never frees them
 * (same contract as CutileGemm's zero-copy views, src/biped/cutile_gemm.rs:
 * 23-27,404-411). Buffers from zl_alloc are freed with zl_free.
 *
 * Matrices are fp32, row-major. Unless stated otherwise a matrix argument
 * has the dense row stride of its logical shape; `ld_*` arguments give an
 * explicit row stride in elements.
 *
 * Threading: one context per host thread (the reference adapter is !Sync,
 * src/biped/cutile_gemm.rs:353-361).
 */
#ifndef ZEALOT_HIP_H
#define ZEALOT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int zl_status;
#define ZL_OK 0
#define ZL_ERR_INVALID 1        /* bad argument (shape, null pointer, range) */
#define ZL_ERR_HIP 2            /* a HIP runtime call failed */
#define ZL_ERR_CODE_OBJECT 3    /* zealot_kernels.hsaco missing or unloadable */
#define ZL_ERR_SELF_TEST 4      /* zl_init's numeric self-test failed */

typedef struct zl_ctx zl_ctx;
typedef struct zl_mlp zl_mlp;
typedef struct zl_ppo zl_ppo;

/* ------------------------------------------------------------ context ---- */

/* Create a context on `device`: one HIP stream, the gfx950 code object loaded
 * with hipModuleLoad, then a numeric self-test against a host fp64 reference
 * (the cases of CutileGemm::self_test, src/biped/cutile_gemm.rs:695-828, at
 * an fp32 tolerance). A non-zero status means "use the fallback path"
 * (CutileGemm::init returning None, src/biped/cutile_gemm.rs:368-424); *out
 * is NULL then and zl_global_error() says why. Setting ZL_FORCE_SELF_TEST_FAIL=1
 * forces the self-test failure branch. */
zl_status zl_init(int device, zl_ctx** out);
void zl_destroy(zl_ctx* ctx);
/* Last error of a call on ctx ("" if none). */
const char* zl_last_error(const zl_ctx* ctx);
/* Error of the last failed zl_init in this process (ctx does not exist). */
const char* zl_global_error(void);
/* The context's hipStream_t, for interop with other HIP code. */
void* zl_stream(zl_ctx* ctx);
/* Worst relative error of the init self-test. */
double zl_self_test_error(const zl_ctx* ctx);
/* Block the host until all work enqueued on ctx has finished. */
zl_status zl_synchronize(zl_ctx* ctx);
/* Version string of the library. */
const char* zl_version(void);
/* Per-launch timing of one kernel of the code object (by its symbol name,
 * e.g. "zk_gemm_am_bn_64x128"): every launch of it on ctx is bracketed by
 * hipEvents on the context stream until zl_timing_end, which returns the summed
 * kernel time, the launch count and, for GEMM variants, the summed algorithmic
 * FLOP (2*M*N*K per GEMM) of those launches. While timing is on, composite entry
 * points launch eagerly instead of replaying their captured graphs. The
 * tracing counterpart of the reference's KHAL_CUDA_PROFILE per-kernel timer
 * (src/bin/iter_e2e_bench.rs:731-735,833-835). */
zl_status zl_timing_begin(zl_ctx* ctx, const char* kernel_name);
zl_status zl_timing_end(zl_ctx* ctx, double* total_ms, long long* launches, double* flops);
/* kernel_name "*" times every kernel; the per-kernel split of the last
 * finished session is then read by kernel index in [0, zl_kernel_count()). */
int zl_kernel_count(void);
zl_status zl_timing_kernel(const zl_ctx* ctx, int index, const char** name, double* total_ms,
                           long long* launches, double* flops);
/* The last finished session's timed launches in issue order: kernel name,
 * milliseconds, algorithmic FLOP and, for GEMMs, shape4 = {M, N, K, split-K
 * slices} (zeros for other kernels). Same timer as above, per launch. */
long long zl_timing_launch_count(const zl_ctx* ctx);
zl_status zl_timing_launch(const zl_ctx* ctx, long long index, const char** name, double* ms,
                           double* flops, int* shape4);
/* sizeof(zl_ppo_config), sizeof(zl_batch), sizeof(zl_ppo_stats) as compiled
 * into the library, for binding generators to check their struct layouts. */
void zl_abi_struct_sizes(size_t out[3]);

/* ------------------------------------------------------------ buffers ---- */

zl_status zl_alloc(zl_ctx* ctx, size_t bytes, void** dev_out);
zl_status zl_free(zl_ctx* ctx, void* dev);
/* Synchronous host <-> device copies on the context stream. */
zl_status zl_upload(zl_ctx* ctx, void* dev_dst, const void* host_src, size_t bytes);
zl_status zl_download(zl_ctx* ctx, void* host_dst, const void* dev_src, size_t bytes);
zl_status zl_copy_d2d(zl_ctx* ctx, void* dev_dst, const void* dev_src, size_t bytes);

/* -------------------------------------- operators (cuTile adapter) ---- */

/* out(m x n) = lhs(m x k) . rhs(k x n). lhs_t: the buffer holds the row-major
 * (k x m) base of lhs; rhs_t: it holds the (n x k) base of rhs. Split-K with a
 * deterministic fixed-order second pass for deep-K, small-output shapes.
 * Replaces CutileGemm::gemm (src/biped/cutile_gemm.rs:477-570). */
zl_status zl_gemm(zl_ctx* ctx, float* out, const float* lhs, int lhs_t, const float* rhs,
                  int rhs_t, int m, int n, int k);

/* out(m x n) = act(lhs(m x k) . rhs(k x n) + bias), bias a column vector read
 * at bias[r * bias_row_stride], act = ELU when elu != 0.
 * Replaces CutileGemm::gemm_bias_act (src/biped/cutile_gemm.rs:578-625). */
zl_status zl_gemm_bias_act(zl_ctx* ctx, float* out, const float* lhs, const float* rhs, int m,
                           int n, int k, const float* bias, int bias_row_stride, int elu);

/* In place g(m x n) *= (y > 0 ? 1 : y + 1), y the post-activation.
 * Replaces CutileGemm::elu_backward (src/biped/cutile_gemm.rs:629-656). */
zl_status zl_elu_backward(zl_ctx* ctx, float* g, const float* y, int m, int n);

/* out(m) = row sums of x(m x n). Replaces CutileGemm::row_sum
 * (src/biped/cutile_gemm.rs:659-690). */
zl_status zl_row_sum(zl_ctx* ctx, float* out, const float* x, int m, int n);

/* ------------------------------------- operators (vortx kernels) ---- */

/* Actor half of the PPO loss for `rows` samples:
 * d_mean = dL/dmean, d_log_std[A] = summed dL/dlog_std (with the entropy
 * term), stats_dev[2] = {sum of scaled surrogate, sum of scaled mean-only KL}
 * (mean_old may be NULL: KL = 0). Semantics of zealot-rl/src/ppo.rs:411-432,
 * 452; replaces vortx Ppo::actor_grad + the dls row_sum
 * (src/bin/biped_train_gpu.rs:1257-1271,1350-1357). All pointers are device
 * pointers. feature_major == 0: mean, action, mean_old and d_mean are
 * batch-major [rows x A] with row strides ld_*; feature_major != 0: they are
 * the trainer's [A x rows] tensors (element (sample r, component k) at
 * ptr[k * ld + r], ld >= rows, e.g. the actor output a[L] and f_act of
 * src/bin/biped_train_gpu.rs:692-694,1055). */
zl_status zl_ppo_actor_grad(zl_ctx* ctx, const float* mean, int ld_mean, const float* action,
                            int ld_action, const float* log_std, const float* adv,
                            const float* logp_old, const float* mean_old, int ld_mean_old,
                            int rows, int action_dim, float clip, float entropy_coef,
                            float scale, float* d_mean, int ld_d_mean, float* d_log_std,
                            float* stats_dev, int feature_major);

/* Critic half: d_v[r] = value_coef * dv * scale with the clipped value loss
 * (zealot-rl/src/ppo.rs:436-450); stats_dev[1] = sum of scaled value loss.
 * Replaces vortx Ppo::value_grad (src/bin/biped_train_gpu.rs:1332-1343). */
zl_status zl_ppo_value_grad(zl_ctx* ctx, const float* v, const float* value_old,
                            const float* ret, int rows, float clip, float value_coef,
                            float scale, float* d_v, float* stats_dev);

/* One Adam step over n elements: the element update of
 * zealot-rl/src/net.rs:240-245 with caller-supplied bias corrections
 * (vortx Adam::step with AdamParams, src/bin/biped_train_gpu.rs:1168-1182). */
zl_status zl_adam_step(zl_ctx* ctx, float* p, const float* g, float* m, float* v, size_t n,
                       float lr, float beta1, float beta2, float eps, float bc1, float bc2);

/* out_dev[0] = sum of squares of x[0..n) (deterministic two-pass).
 * Replaces vortx Reduce::SqNorm (src/bin/biped_train_gpu.rs:1377-1397). */
zl_status zl_grad_sqnorm(zl_ctx* ctx, const float* x, size_t n, float* out_dev);

/* A device tensor of n floats (one gradient tensor of the trainer's
 * per-tensor buffers: net.dw[l], net.db[l], dls). */
typedef struct zl_tensor {
  const float* ptr;
  size_t n;
} zl_tensor;

/* The trainer's global grad-norm clip without the host round trip
 * (src/bin/biped_train_gpu.rs:1368-1452: Reduce::SqNorm per tensor, the
 * readback, the norm, OpAssign::Mul): norm = sqrt(sum over the `count`
 * tensors of their sums of squares), fixed summation order;
 * scale_dev[0] = max_norm / norm when max_norm > 0 and norm > max_norm, else
 * 1; norm_dev[0] = norm (norm_dev may be NULL). Gradients are not modified:
 * zl_adam_multi applies the scale. count <= 48. Asynchronous; device
 * outputs. */
zl_status zl_grad_clip_scale(zl_ctx* ctx, const zl_tensor* tensors, int count, float max_norm,
                             float* scale_dev, float* norm_dev);

/* zl_grad_clip_scale without any allocation: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, serving or training loops that forbid hipMalloc). Same results,
 * bit for bit, as zl_grad_clip_scale. Its partial sums live in a static
 * device array per GPU (256 KiB, held until the process ends) of 4 slots of
 * 16,384 floats: one partial per 2,048 elements of each tensor (at least one
 * per tensor), so about 33.5 M gradient elements per call at most; larger
 * inputs are refused with ZL_ERR_INVALID. zl_init claims one slot for the
 * context and zl_destroy returns it: the calls of one context are ordered on
 * its stream and never share partials with another context's. With 4
 * contexts alive on a GPU, a fifth gets ZL_ERR_INVALID from this entry point
 * (its other entry points work) until one is destroyed. Each call leaves its
 * slot holding its partials; nothing needs clearing between calls. */
zl_status zl_grad_clip_scale_noalloc(zl_ctx* ctx, const zl_tensor* tensors, int count,
                                     float max_norm, float* scale_dev, float* norm_dev);

/* One Adam parameter tensor with its gradient and moments (device, n floats each). */
typedef struct zl_adam_tensor {
  float* p;
  const float* g;
  float* m;
  float* v;
  size_t n;
} zl_adam_tensor;

/* One Adam step over `count` tensors in one launch (vortx Adam::step per
 * tensor with AdamParams, src/bin/biped_train_gpu.rs:501-538,1453-1461;
 * element update of zealot-rl/src/net.rs:240-245), each gradient multiplied
 * by clip_scale_dev[0] first (a device scalar, e.g. from zl_grad_clip_scale;
 * NULL: 1). count <= 48. Asynchronous. */
zl_status zl_adam_multi(zl_ctx* ctx, const zl_adam_tensor* tensors, int count, float lr,
                        float beta1, float beta2, float eps, float bc1, float bc2,
                        const float* clip_scale_dev);

/* The trainer's whole clipped optimiser step (src/bin/biped_train_gpu.rs:
 * 1368-1461: Reduce::SqNorm per gradient tensor, the global norm and clip
 * scale, Adam::step per tensor) in two launches instead of three: the sums
 * of squares of the tensors' gradients, then one Adam launch whose blocks
 * each take the clip scale from them (max_norm / norm when max_norm > 0 and
 * norm > max_norm, else 1). Bit-identical to zl_grad_clip_scale over the
 * gradients followed by zl_adam_multi with its scale. scale_dev[0] and
 * norm_dev[0] receive the scale and the norm (either may be NULL). count <=
 * 48. Asynchronous. */
zl_status zl_adam_multi_clip(zl_ctx* ctx, const zl_adam_tensor* tensors, int count, float lr,
                             float beta1, float beta2, float eps, float bc1, float bc2,
                             float max_norm, float* scale_dev, float* norm_dev);

/* GAE(lambda) for N independent trajectories of length T, one lane per env
 * (zealot-rl/src/ppo.rs:681-703, run per env by
 * src/bin/biped_train_gpu.rs:974-981). Element (t, e) of rewards / values /
 * dones is at t*in_ts + e*in_es, of adv / ret at t*out_ts + e*out_es;
 * last_values[e] bootstraps the final step; dones are 0/1 bytes. */
zl_status zl_gae(zl_ctx* ctx, const float* rewards, const float* values, const uint8_t* dones,
                 const float* last_values, int T, int N, long long in_ts, long long in_es,
                 long long out_ts, long long out_es, float gamma, float lam, float* adv,
                 float* ret);

/* In place (adv - mean) / max(sqrt(population var), 1e-6)
 * (zealot-rl/src/ppo.rs:343-348, src/bin/biped_train_gpu.rs:1010-1016). */
zl_status zl_adv_normalize(zl_ctx* ctx, float* adv, size_t n);

/* action = mean + exp(log_std) * eps, logp = Gaussian log-prob of action
 * (ActorCritic::sample / logp, zealot-rl/src/ppo.rs:297-323; the host loop of
 * src/bin/biped_train_gpu.rs:910-930), eps supplied by the caller. */
zl_status zl_sample_actions(zl_ctx* ctx, const float* mean, int ld_mean, const float* log_std,
                            const float* eps, int rows, int action_dim, float* action,
                            float* logp);

/* ----------------------------------------- observation normalisation ---- */

/* A running normaliser lives in device memory as float[2 * dim + 1]:
 * mean[dim], m2[dim], count (Normalizer, zealot-rl/src/ppo.rs:104-113). A
 * pending state (PendingNorm, :115-122) has the same layout; count 0 means
 * empty. dim <= 4096. All calls are enqueued on the context's stream. */

/* unit_prior != 0: Normalizer::new (ppo.rs:141-148: mean 0, m2 1, count 1);
 * unit_prior == 0: an empty PendingNorm (PendingNorm::default). */
zl_status zl_norm_reset(zl_ctx* ctx, float* state, int dim, int unit_prior);
/* Fold rows x[r * ld + i], r = 0 .. rows-1 in order, into a state:
 * Normalizer::update (ppo.rs:161-168, ActorCritic::record_obs :276-279) on a
 * live state, PendingNorm::push (:126-137) on a pending one. count is exact
 * (the reference's f32 `count += 1.0`, saturating at 2^24); mean and m2 are
 * folded in chunks of 256 rows and agree with the one-at-a-time fold to fp32
 * rounding. */
zl_status zl_norm_update(zl_ctx* ctx, float* state, int dim, const float* x, int ld,
                         long long rows);
/* Normalizer::commit (ppo.rs:179-195): merge pending into state (Chan), then
 * empty pending; no-op when pending is empty. */
zl_status zl_norm_commit(zl_ctx* ctx, float* state, float* pending, int dim);
/* Normalizer::normalize (ppo.rs:198-205) of each row:
 * out[r * ld_out + i] = clamp((x[r * ld_x + i] - mean[i]) / sqrt(max(m2[i] / count, 1e-8)), -5, 5).
 * out may be x (in place) when ld_out == ld_x. */
zl_status zl_norm_normalize(zl_ctx* ctx, const float* state, int dim, const float* x, int ld_x,
                            long long rows, float* out, int ld_out);

/* ------------------------------------------------ GpuMlp equivalent ---- */

/* A dense ELU MLP (hidden ELU, linear output) with device-resident weights,
 * Adam moments and activation buffers for up to `batch` rows: the GpuMlp of
 * src/bin/biped_train_gpu.rs:316-564. zl_mlp_create takes the caller's
 * input, output and output gradient batch-major ([rows x dim], a row stride). */
zl_status zl_mlp_create(zl_ctx* ctx, const int* dims, int ndims, int batch, zl_mlp** out);
/* flags = ZL_MLP_FEATURE_MAJOR: the input x, the output and the output
 * gradient are feature-major [dim x rows] with a feature stride ld >= rows
 * (element (row r, feature f) at f * ld + r), as GpuMlp keeps a[0], a[L] and
 * delta[L-1] ([d[i] x m], src/bin/biped_train_gpu.rs:351-355, used as W.a at
 * :382-394 and over delta at :436-492). Results are bit-identical to the
 * batch-major handle given the same values at 16-byte aligned strides. */
#define ZL_MLP_FEATURE_MAJOR 1
zl_status zl_mlp_create_ex(zl_ctx* ctx, const int* dims, int ndims, int batch, int flags,
                           zl_mlp** out);
void zl_mlp_destroy(zl_mlp* mlp);
/* Number of parameters in the packed layout w[0], b[0], w[1], b[1], ... with
 * w[l] row-major [dims[l+1] x dims[l]] (zealot-rl/src/net.rs:30-34). */
long long zl_mlp_num_params(const zl_mlp* mlp);
/* Host packed params <-> device (GpuMlp::write_w / read_into, :541-563). */
zl_status zl_mlp_write_weights(zl_mlp* mlp, const float* packed_host);
zl_status zl_mlp_read_weights(zl_mlp* mlp, float* packed_host);
/* Forward over `rows` input rows (device x; batch-major: row stride
 * ldx >= dims[0]; feature-major: feature stride ldx >= rows): all layer
 * activations stay resident for zl_mlp_backward (GpuMlp::forward, :364-422).
 * A batch-major x is borrowed (read again by zl_mlp_backward, as GpuMlp
 * reads a[0]) and must stay valid until then; a feature-major x is staged
 * into the handle's own buffer and may be released after the call. */
zl_status zl_mlp_forward(zl_mlp* mlp, const float* x, int ldx, int rows);
/* Device pointer to the output activations of the last forward and their
 * stride: [rows x dims[L]] (row stride) or, feature-major, [dims[L] x rows]
 * (feature stride; GpuMlp's a[L]). Owned by the handle. */
const float* zl_mlp_output(const zl_mlp* mlp, int* ld_out);
/* Backward of dL/dout (device; batch-major [rows x dims[L]] with row stride
 * ld_g, or feature-major [dims[L] x rows] with feature stride ld_g >= rows)
 * through the last forward: weight/bias gradients summed over the rows
 * (GpuMlp::backward, :423-500). */
zl_status zl_mlp_backward(zl_mlp* mlp, const float* g_out, int ld_g);
/* Download the gradients of the last backward, packed like the params. */
zl_status zl_mlp_read_grads(zl_mlp* mlp, float* packed_host);
/* Adam over all tensors with caller bias corrections (GpuMlp::adam, :501-538). */
zl_status zl_mlp_adam(zl_mlp* mlp, float lr, float bc1, float bc2);
/* Download / upload the Adam moments, packed like the params. */
zl_status zl_mlp_read_moments(zl_mlp* mlp, float* m_host, float* v_host);
zl_status zl_mlp_write_moments(zl_mlp* mlp, const float* m_host, const float* v_host);

/* ----------------------------------------------- the PPO update ---- */

#define ZL_SEMANTICS_ACTOR_CRITIC 0 /* ActorCritic::update, zealot-rl/src/ppo.rs:338-510 */
#define ZL_SEMANTICS_GPU_TRAINER 1  /* src/bin/biped_train_gpu.rs:1164-1553 */

typedef struct zl_ppo_config {
  int semantics;       /* ZL_SEMANTICS_* */
  float clip;          /* surrogate and value clip (PpoConfig::clip) */
  float entropy_coef;
  float value_coef;
  int epochs;
  int minibatches;
  /* ACTOR_CRITIC: MlpGrad::clip per net (log_std unclipped).
   * GPU_TRAINER: global norm over actor + critic + log_std, <= 0 disables. */
  float max_grad_norm;
  float desired_kl;
  float lr_min, lr_max;
  int adaptive_lr;     /* per minibatch (ACTOR_CRITIC) or per epoch (GPU_TRAINER) */
  int early_stop;      /* GPU_TRAINER: stop epochs once KL > 5 * desired_kl */
  int shuffle;         /* ACTOR_CRITIC: per-epoch Fisher-Yates (ppo.rs:357-363); else contiguous */
  int normalize_adv;   /* normalise advantages in place first */
  int clamp_log_std;   /* ACTOR_CRITIC: [-1.6, 1.0] each step; GPU_TRAINER: [-1.6, 0.0] after */
} zl_ppo_config;

/* Layout bits of zl_batch.feature_major: the field is the trainer's
 * feature-major [dim x n] tensor (element (sample i, feature k) at
 * ptr[k * ld + i], ld >= n: f_obs / f_cobs / f_act of
 * src/bin/biped_train_gpu.rs:1029-1030,1053-1056) instead of batch-major
 * [n x dim] rows (ptr[i * ld + k]). */
#define ZL_FM_OBS 1u
#define ZL_FM_CRITIC_OBS 2u
#define ZL_FM_ACTION 4u
#define ZL_FM_MEAN_OLD 8u

/* One rollout batch, structure of arrays, all DEVICE pointers, n samples in
 * batch order (sample i = column / row i). obs and critic_obs are the already
 * normalised observations (the trainer stages normalised obs,
 * src/bin/biped_train_gpu.rs:1021-1030). The update copies the batch into
 * its own buffers at its start (inside the same graph replay), so the
 * buffers may change from call to call without a re-capture; they must stay
 * valid until the call returns. */
typedef struct zl_batch {
  long long n;
  const float* obs;        int ld_obs;       /* [n x actor_dims[0]] */
  const float* critic_obs; int ld_critic_obs;/* [n x critic_dims[0]] (may alias obs) */
  const float* action;     int ld_action;    /* [n x A] */
  const float* mean_old;   int ld_mean_old;  /* [n x A] rollout means (KL), may be NULL */
  const float* logp_old;                     /* [n] */
  const float* value_old;                    /* [n] */
  float* adv;                                /* [n], normalised in place if requested */
  const float* ret;                          /* [n] */
  unsigned feature_major;                    /* ZL_FM_* bits; 0 = all batch-major */
} zl_batch;

/* PpoStats (zealot-rl/src/ppo.rs:90-102) plus the trainer's epoch count. */
typedef struct zl_ppo_stats {
  float kl, surrogate, value_loss, entropy, lr;
  int epochs_run;
  float last_kl;       /* GPU_TRAINER: last per-epoch full-Gaussian KL */
  float grad_norm[3];  /* last pre-clip norms: actor, critic, log_std (global in [0]) */
} zl_ppo_stats;

/* Actor + critic + log_std and their Adam state resident in one flat HBM
 * buffer; activation / gradient buffers sized for `minibatch_rows` rows. The
 * ActorCritic of zealot-rl/src/ppo.rs:208-229 with the trainer's GpuMlp pair. */
zl_status zl_ppo_create(zl_ctx* ctx, const int* actor_dims, int n_actor, const int* critic_dims,
                        int n_critic, int minibatch_rows, zl_ppo** out);
void zl_ppo_destroy(zl_ppo* ppo);
/* Host packed params (as zl_mlp_write_weights) <-> device; lr is the current
 * adaptive learning rate. zl_ppo_set_params resets nothing else. */
zl_status zl_ppo_set_params(zl_ppo* ppo, const float* actor, const float* critic,
                            const float* log_std, float lr);
zl_status zl_ppo_get_params(zl_ppo* ppo, float* actor, float* critic, float* log_std, float* lr);
/* Adam moments, packed (any pointer may be NULL). */
zl_status zl_ppo_get_moments(zl_ppo* ppo, float* m_actor, float* v_actor, float* m_critic,
                             float* v_critic, float* m_log_std, float* v_log_std);
/* Zero the Adam moments and step counters (a freshly constructed ActorCritic). */
zl_status zl_ppo_reset_optimizer(zl_ppo* ppo);
/* Adam step count (ACTOR_CRITIC t) and trainer gstep. */
zl_status zl_ppo_get_counters(zl_ppo* ppo, int* t, unsigned long long* gstep);
/* The whole update: epochs x minibatches of actor + critic forward, PPO losses,
 * backward, grad clip, Adam, adaptive LR, all on the device with no host
 * round trip inside (captured once into a hipGraph and replayed). Blocks until
 * done and fills *stats (ActorCritic::update, zealot-rl/src/ppo.rs:338-384, or
 * src/bin/biped_train_gpu.rs:1164-1553 per config->semantics). */
zl_status zl_ppo_update(zl_ppo* ppo, const zl_batch* batch, const zl_ppo_config* config,
                        zl_ppo_stats* stats);
/* Captured update graphs of this handle so far and the host time of the last
 * capture + instantiation (milliseconds). A graph is re-captured only when the
 * update's shapes, strides, layouts or configuration change, or when a buffer
 * it uses had to grow; new batch pointers alone never re-capture. */
zl_status zl_ppo_graph_info(zl_ppo* ppo, long long* captures, double* last_capture_ms);
/* Gradients of one minibatch without stepping: forward, PPO losses and
 * backward over batch rows [row0, row0 + rows) (or rows perm_dev[row0 + r] when
 * perm_dev, a device int array whose entries are in [0, n), is non-NULL;
 * row0 + rows <= n either way), leaving the summed gradients in
 * the flat gradient buffer (read them with zl_ppo_get_grads) and
 * stats[3] = {surrogate, value_loss, kl} (host). The accumulation of
 * zealot-rl/src/ppo.rs:406-462 before clip / Adam. Blocks until done. */
zl_status zl_ppo_minibatch_grads(zl_ppo* ppo, const zl_batch* batch, const zl_ppo_config* config,
                                 long long row0, int rows, const int* perm_dev, float* stats);
/* Download the gradient buffer, packed like the params (any pointer may be NULL). */
zl_status zl_ppo_get_grads(zl_ppo* ppo, float* actor, float* critic, float* log_std);
/* One rollout step for n envs on the device: GpuPolicy::forward
 * (src/biped/gpu_policy.rs:210-248) and the trainer's sampling loop
 * (src/bin/biped_train_gpu.rs:910-930) without the host round trip. Row r of
 * obs (and critic_obs) is normalised with its normaliser state (as
 * zl_norm_normalize; a NULL state means the rows are already normalised),
 * then mean = actor(obs_r), action[r * A + k] = mean_k + exp(log_std_k) *
 * eps[r * A + k], logp[r] = ActorCritic::logp(action, mean) (ppo.rs:297-306)
 * and value[r] = critic(critic_obs_r). mean (row stride ld_mean) and value
 * may be NULL; critic_obs and critic_norm are only read when value is not
 * NULL. Asynchronous on the context's stream.
 * Launch forms (same results either way): up to 8,192 rows, when the nets
 * used fit, the whole step is ONE zk_policy launch (normalise, every layer
 * with the activations in LDS, sampling, logp, value). A net fits when it
 * has at most 8 layers, input and hidden widths up to 512 with hidden widths
 * multiples of 16, at most 32 outputs, and layer-0 weight rows padded to a
 * multiple of 16 (the handle pads them itself when that adds at most 1/8,
 * e.g. 123 -> 128). Otherwise, and for larger n, the rows go through the
 * layer GEMMs in minibatch-sized chunks with separate normalise and sampling
 * launches. The environment variable ZL_POLICY_FUSED=0 (read at zl_init)
 * turns the single-launch form off; zl_ppo_values and zl_ppo_actor_mean
 * follow the same rule per net. The single launch reads the weights from a
 * second, fragment-major copy held by the handle (about the size of the
 * weights), which zl_ppo_create, zl_ppo_set_params, zl_ppo_load* and every
 * zl_ppo_update rewrite on the stream after changing the parameters. */
zl_status zl_ppo_act(zl_ppo* ppo, const float* obs_norm, const float* obs, int ld_obs,
                     const float* critic_norm, const float* critic_obs, int ld_critic_obs,
                     long long n, const float* eps, float* action, float* logp, float* mean,
                     int ld_mean, float* value);
/* ActorCritic::save (zealot-rl/src/ppo.rs:512-570): a .safetensors image with
 * the reference's tensors (all F32) "actor.w_{l}" [out, in], "actor.b_{l}"
 * [out], "critic.*" likewise, "log_std" [A], "obs_norm.mean" / ".m2" [dim],
 * "obs_norm.count" [1], "critic_norm.*" likewise and "lr" [1]. obs_norm /
 * critic_norm are normaliser states (zl_norm_*); NULL saves Normalizer::new.
 * with_optimizer != 0 also writes the Adam moments ("adam_m.<net>.w_{l}",
 * "adam_v.*", "adam_m.log_std", "adam_v.log_std", F32) and the step counters
 * ("adam.t", "adam.gstep", I64 [1]), which the reference's load ignores.
 * Blocks until the device state is read. */
zl_status zl_ppo_save(zl_ppo* ppo, const float* obs_norm, const float* critic_norm,
                      int with_optimizer, const char* path);
/* The same image in memory: *size gets its byte count; buf may be NULL to
 * query the size only; otherwise cap must be >= *size. */
zl_status zl_ppo_save_bytes(zl_ppo* ppo, const float* obs_norm, const float* critic_norm,
                            int with_optimizer, void* buf, size_t cap, size_t* size);
/* ActorCritic::load / load_from_bytes (ppo.rs:572-650) into an existing
 * handle whose net dims equal the file's (zl_checkpoint_dims reads them):
 * params, log_std, lr, and the normaliser states into obs_norm / critic_norm
 * (NULL skips one). The Adam state is reset as the reference's load does,
 * unless restore_optimizer != 0 and the image carries the "adam.*" tensors,
 * which are then restored. Tensors the loader reads must be F32 (I64 for the
 * counters). Blocks until done. */
zl_status zl_ppo_load(zl_ppo* ppo, float* obs_norm, float* critic_norm, int restore_optimizer,
                      const char* path);
zl_status zl_ppo_load_bytes(zl_ppo* ppo, float* obs_norm, float* critic_norm,
                            int restore_optimizer, const void* buf, size_t size);
/* Net dims of a checkpoint image (the reference's load reconstructs them from
 * the weight shapes, ppo.rs:585-610): n_actor / n_critic get the counts;
 * actor_dims / critic_dims (may be NULL) get the dims when count <= cap.
 * Host only, no context; errors via zl_global_error. */
zl_status zl_checkpoint_dims(const void* buf, size_t size, int* actor_dims, int* n_actor,
                             int* critic_dims, int* n_critic, int cap);
/* Critic values for n rows of (normalised) critic obs, in minibatch-sized
 * chunks: values[i] (ActorCritic::value, zealot-rl/src/ppo.rs:290-294). */
zl_status zl_ppo_values(zl_ppo* ppo, const float* critic_obs, int ld, long long n,
                        float* values);
/* Actor means for n rows of (normalised) obs: mean[i * ld_mean + k]
 * (ActorCritic::mean, zealot-rl/src/ppo.rs:282-287; GpuPolicy::forward,
 * src/biped/gpu_policy.rs:210-248). */
zl_status zl_ppo_actor_mean(zl_ppo* ppo, const float* obs, int ld, long long n, float* mean,
                            int ld_mean);

#ifdef __cplusplus
}
#endif

#endif /* ZEALOT_HIP_H */
