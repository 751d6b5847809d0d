// zl_oracle.hpp — CPU restatement of zealot-rl's learning tier.
//
// TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
// path and the timed CPU baseline. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it; the product path never does.
//
// It restates, in scalar C++ with FP contraction off, the reference files
//   zealot-rl/src/rng.rs   (Lcg, Box-Muller gauss)
//   zealot-rl/src/net.rs   (Mlp, MlpGrad, Adam)
//   zealot-rl/src/ppo.rs   (Normalizer, ActorCritic, gae, update)
// and the GPU trainer's update semantics from
//   src/bin/biped_train_gpu.rs:1164-1553
// Each function cites the lines it follows. Operation order is kept exactly
// (left-associative f32 arithmetic, bias-first accumulation, libm expf/logf/
// cosf, correctly rounded sqrtf, square-and-multiply powi) so results are
// bit-identical to the Rust code wherever that code is deterministic. The one
// place it is not (rayon fold/reduce grouping, ppo.rs:406-462) is restated as
// contiguous per-thread chunks reduced left to right; with one thread this is
// the sequential fold.
//
// Pinning: every function used by the tests is checked against the
// reference's own known-answer tests, closed forms or float64 finite
// differences (tests/test_oracle.py); the normaliser (Normalizer::update,
// PendingNorm::push, norm_commit, normalize; ppo.rs:104-206) by the float64
// Chan-merge closed forms, the unit-prior identity, the variance floor and
// the f32 count saturation at 2^24; the GPU trainer's optimiser branch
// (trainer_update: global clip over actor + critic + log_std, bias correction
// from the epoch's shared gstep) and the minibatch / epoch statistics
// (surrogate, value loss, mean-only KL, entropy) by a float64 restatement of
// the epoch built from tests/np_ref.py, which also shows that log_std left out
// of the norm, a per-net clip or a per-minibatch Adam t fail the check.
#pragma once
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <vector>

namespace zlo {

// std::f32::consts::TAU rounded to f32.
constexpr float kTau = 6.28318530717958647692f;
// ppo.rs:18 LOG_SQRT_2PI
constexpr float kLogSqrt2Pi = 0.9189385f;

// Rust `f32::powi` lowers to the libgcc/compiler-rt __powisf2 loop: square and
// multiply from the low bit up, plain f32 multiplies (net.rs:237-238).
float powi_f32(float x, int n);

// rng.rs:9-31
struct Lcg {
  uint64_t s;
  explicit Lcg(uint64_t seed) : s(seed | 1ULL) {}
  float unit() {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    return (float)(s >> 40) / (float)(1ULL << 24);
  }
  float gauss() {
    // Rust evaluates the left factor (using u1) before drawing u2.
    float u1 = std::fmax(unit(), 1e-7f);
    float a = std::sqrt(-2.0f * std::log(u1));
    float u2 = unit();
    return a * std::cos(kTau * u2);
  }
};

// net.rs:14-23
inline float elu(float x) { return x > 0.0f ? x : std::exp(x) - 1.0f; }
inline float elu_grad_from_act(float a) { return a > 0.0f ? 1.0f : a + 1.0f; }

struct MlpGrad;

// net.rs:27-35. w[l] is row-major [dims[l+1] x dims[l]].
struct Mlp {
  std::vector<size_t> dims;
  std::vector<std::vector<float>> w, b;

  Mlp() = default;
  // net.rs:61-79: w ~ N(0, 1/fan_in) from the Lcg, last layer x out_scale, b = 0.
  static Mlp create(const std::vector<size_t>& dims, float out_scale, Lcg& rng);
  size_t layers() const { return w.size(); }
  // net.rs:88-108. acts[0] = x, acts[L] = output.
  void forward(const float* x, std::vector<std::vector<float>>& acts) const;
  // net.rs:113-140. Accumulates into g, returns dL/dx in gin (if non-null).
  void backward(const std::vector<std::vector<float>>& acts, const float* g_out, MlpGrad& g,
                std::vector<float>* gin) const;
  size_t num_params() const;
  // Packed layout used across the C ABI: for l: w[l] then b[l].
  void pack(float* out) const;
  void unpack(const float* in);
};

// net.rs:38-43, 145-203
struct MlpGrad {
  std::vector<std::vector<float>> w, b;
  static MlpGrad zero(const Mlp& net);
  void add(const MlpGrad& o);
  void scale(float s);
  float l2_norm() const;
  void clip(float max_norm);
  void pack(float* out) const;
  void unpack(const float* in);
};

// net.rs:207-252
struct Adam {
  std::vector<std::vector<float>> mw, vw, mb, vb;
  int t = 0;
  float beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f;
  static Adam create(const Mlp& net);
  void step(Mlp& net, const MlpGrad& g, float lr);
};

// The Adam element update of net.rs:240-245, shared by every restated caller.
inline void adam_elem(float& p, float gr, float& m, float& v, float lr, float b1, float b2,
                      float bc1, float bc2, float eps) {
  m = b1 * m + (1.0f - b1) * gr;
  v = b2 * v + (1.0f - b2) * gr * gr;
  p -= lr * (m / bc1) / (std::sqrt(v / bc2) + eps);
}

// ppo.rs:104-206
struct Normalizer {
  std::vector<float> mean, m2;
  float count = 1.0f;
  static Normalizer create(size_t dim);
  void update(const float* x);
  void normalize(const float* x, float* out) const;
};

struct PendingNorm {
  std::vector<float> mean, m2;
  float count = 0.0f;
  void push(const float* x, size_t dim);
};
void norm_commit(Normalizer& n, PendingNorm& p);

// ppo.rs:22-65
struct PpoConfig {
  float gamma = 0.99f, lam = 0.95f, clip = 0.2f, entropy_coef = 0.01f, value_coef = 1.0f;
  int epochs = 5, minibatches = 4;
  float max_grad_norm = 1.0f, desired_kl = 0.01f;
  float lr_min = 1e-5f, lr_max = 1e-2f;
  bool adaptive_lr = true;
};

// ppo.rs:90-102
struct PpoStats {
  float kl = 0, surrogate = 0, value_loss = 0, entropy = 0, lr = 0;
};

// ppo.rs:69-87, stored as structure-of-arrays over n samples.
struct Batch {
  size_t n = 0, od = 0, cd = 0, ad = 0;
  const float* obs = nullptr;         // [n x od]
  const float* critic_obs = nullptr;  // [n x cd]
  const float* action = nullptr;      // [n x ad]
  const float* mean_old = nullptr;    // [n x ad]
  const float* logp_old = nullptr;    // [n]
  const float* value_old = nullptr;   // [n]
  float* adv = nullptr;               // [n] (normalised in place by update)
  const float* ret = nullptr;         // [n]
};

// ppo.rs:208-229
struct ActorCritic {
  Mlp actor, critic;
  std::vector<float> log_std;
  Normalizer obs_norm, critic_norm;
  Adam opt_actor, opt_critic;
  std::vector<float> m_logstd, v_logstd;
  int t_logstd = 0;
  float lr = 1e-3f;

  // ppo.rs:235-266
  static ActorCritic create(const std::vector<size_t>& actor_dims,
                            const std::vector<size_t>& critic_dims, float init_noise_std,
                            float init_lr, Lcg& rng);
  size_t action_dim() const { return log_std.size(); }
  void mean(const float* obs, float* out) const;              // ppo.rs:282-287
  float value(const float* critic_obs) const;                 // ppo.rs:290-294
  float logp(const float* action, const float* mean) const;   // ppo.rs:297-305
  float entropy() const;                                      // ppo.rs:308-311
  float sample(const float* obs, Lcg& rng, float* action, float* mean) const;  // ppo.rs:314-323
  float kl(const float* mean_new, const float* mean_old) const;  // ppo.rs:327-334
  // ppo.rs:338-384. `nthreads` workers fold contiguous chunks of each
  // minibatch (rayon analogue); `normalize_obs=false` means the batch obs are
  // already normalised (the GPU trainer stages normalised obs).
  PpoStats update(Batch& batch, const PpoConfig& cfg, int nthreads, bool normalize_obs);
  // ppo.rs:388-493
  PpoStats minibatch_step(const Batch& batch, const size_t* idx, size_t count,
                          const PpoConfig& cfg, int nthreads, bool normalize_obs);
  void step_log_std(const float* g);  // ppo.rs:496-510
};

// ppo.rs:681-703
void gae(const float* rewards, const float* values, const uint8_t* dones, size_t t,
         float last_value, float gamma, float lam, float* adv, float* ret);

// The GPU trainer's update (src/bin/biped_train_gpu.rs:1164-1553), restated on
// the CPU: contiguous minibatches (no shuffle), global grad-norm clip over
// actor + critic + log_std, Adam bias correction from the per-epoch `gstep`,
// per-epoch full-Gaussian KL on the last minibatch driving the adaptive LR and
// early stop, log_std unclamped during the update and clamped to
// [-1.6, 0.0] after it.
struct TrainerState {
  Mlp actor, critic;
  std::vector<float> log_std;
  // Adam moments, packed like Mlp::pack.
  std::vector<float> ma, va, mc, vc, mls, vls;
  uint64_t gstep = 0;
  float lr = 1e-3f;
};

struct TrainerConfig {
  float clip = 0.2f, entropy_coef = 0.01f, value_coef = 1.0f;
  int epochs = 5, minibatches = 4;
  float grad_clip = 1.0f;  // <= 0 disables
  float desired_kl = 0.01f, lr_min = 1e-5f, lr_max = 1e-2f;
  bool adaptive_lr = true;
  bool early_stop = true;
  bool clamp_after = true;  // biped_train_gpu.rs:1529-1541
};

struct TrainerResult {
  PpoStats stats;
  int epochs_run = 0;
  float last_kl = 0;
};

// Gradients of one minibatch over explicit sample indices, without clip or
// Adam (the fold/reduce of ppo.rs:406-462). obs are already normalised.
// stats = {surrogate, value_loss, kl} sums (scaled by 1/count).
void minibatch_grads(const Mlp& actor, const Mlp& critic, const std::vector<float>& log_std,
                     const Batch& batch, const size_t* idx, size_t count, float clip,
                     float entropy_coef, float value_coef, int nthreads, MlpGrad& ga, MlpGrad& gc,
                     std::vector<float>& gls, float stats[3]);

// Runs one update. obs/critic_obs are already normalised (staged layout).
TrainerResult trainer_update(TrainerState& st, const Batch& batch, const TrainerConfig& cfg,
                             int nthreads);

}  // namespace zlo
