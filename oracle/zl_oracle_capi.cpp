// zl_oracle_capi.cpp — extern "C" surface of the CPU oracle for ctypes.
// TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py, never by the product path.
//
// Nets cross this boundary in the packed layout w[0], b[0], w[1], b[1], ...
// with w[l] row-major [dims[l+1] x dims[l]] (zealot-rl/src/net.rs:30-34).
#include <cstring>
#include <vector>

#include "zl_oracle.hpp"

using namespace zlo;

namespace {
std::vector<size_t> to_dims(const int* d, int n) {
  std::vector<size_t> v(n);
  for (int i = 0; i < n; ++i) v[i] = (size_t)d[i];
  return v;
}
Mlp make_net(const int* dims, int ndims, const float* params) {
  Lcg dummy(1);
  Mlp net = Mlp::create(to_dims(dims, ndims), 1.0f, dummy);
  if (params) net.unpack(params);
  return net;
}
}  // namespace

extern "C" {

struct zlo_ppo_cfg {
  float gamma, lam, clip, entropy_coef, value_coef;
  int epochs, minibatches;
  float max_grad_norm, desired_kl, lr_min, lr_max;
  int adaptive_lr;
};

struct zlo_trainer_cfg {
  float clip, entropy_coef, value_coef;
  int epochs, minibatches;
  float grad_clip, desired_kl, lr_min, lr_max;
  int adaptive_lr, early_stop, clamp_after;
};

void zlo_lcg_units(uint64_t seed, int n, float* out) {
  Lcg r(seed);
  for (int i = 0; i < n; ++i) out[i] = r.unit();
}

void zlo_lcg_gauss(uint64_t seed, int n, float* out) {
  Lcg r(seed);
  for (int i = 0; i < n; ++i) out[i] = r.gauss();
}

float zlo_powi(float x, int n) { return powi_f32(x, n); }

float zlo_elu(float x) { return elu(x); }
float zlo_elu_grad_from_act(float a) { return elu_grad_from_act(a); }

// Mlp::new(dims, out_scale, &mut Lcg::new(seed)) -> packed params.
void zlo_mlp_init(const int* dims, int ndims, float out_scale, uint64_t seed, float* params) {
  Lcg r(seed);
  Mlp net = Mlp::create(to_dims(dims, ndims), out_scale, r);
  net.pack(params);
}

// Per-row Mlp::forward over M rows. acts_out holds a[1..=L] back to back, each
// [M x dims[l]] row-major.
void zlo_mlp_forward(const int* dims, int ndims, const float* params, const float* x, int M,
                     float* acts_out) {
  Mlp net = make_net(dims, ndims, params);
  std::vector<std::vector<float>> a;
  std::vector<size_t> off(ndims, 0);
  for (int l = 2; l < ndims; ++l) off[l] = off[l - 1] + (size_t)M * dims[l - 1];
  for (int r = 0; r < M; ++r) {
    net.forward(x + (size_t)r * dims[0], a);
    for (int l = 1; l < ndims; ++l)
      std::memcpy(acts_out + off[l] + (size_t)r * dims[l], a[l].data(), dims[l] * 4);
  }
}

// Per-row Mlp::backward over M rows in order, accumulating into one MlpGrad
// (the sequential fold). grads_out is packed; gin_out [M x dims[0]] may be NULL.
void zlo_mlp_backward(const int* dims, int ndims, const float* params, const float* x, int M,
                      const float* g_out, float* grads_out, float* gin_out) {
  Mlp net = make_net(dims, ndims, params);
  MlpGrad g = MlpGrad::zero(net);
  std::vector<std::vector<float>> a;
  std::vector<float> gin;
  int out = dims[ndims - 1];
  for (int r = 0; r < M; ++r) {
    net.forward(x + (size_t)r * dims[0], a);
    net.backward(a, g_out + (size_t)r * out, g, gin_out ? &gin : nullptr);
    if (gin_out) std::memcpy(gin_out + (size_t)r * dims[0], gin.data(), dims[0] * 4);
  }
  g.pack(grads_out);
}

// MlpGrad::clip on a packed gradient; returns the pre-clip l2_norm.
float zlo_mlpgrad_clip(const int* dims, int ndims, float* g_packed, float max_norm) {
  Mlp net = make_net(dims, ndims, nullptr);
  MlpGrad g = MlpGrad::zero(net);
  g.unpack(g_packed);
  float n = g.l2_norm();
  g.clip(max_norm);
  g.pack(g_packed);
  return n;
}

// Adam::step for a packed net whose optimiser has already taken t-1 steps.
void zlo_adam_step(const int* dims, int ndims, float* p, const float* g, float* m, float* v,
                   int t, float lr) {
  Mlp net = make_net(dims, ndims, p);
  MlpGrad gr = MlpGrad::zero(net);
  gr.unpack(g);
  Adam opt = Adam::create(net);
  // Load moments (packed like the params).
  MlpGrad mm = MlpGrad::zero(net), vv = MlpGrad::zero(net);
  mm.unpack(m);
  vv.unpack(v);
  opt.mw = mm.w;
  opt.mb = mm.b;
  opt.vw = vv.w;
  opt.vb = vv.b;
  opt.t = t - 1;
  opt.step(net, gr, lr);
  net.pack(p);
  mm.w = opt.mw;
  mm.b = opt.mb;
  vv.w = opt.vw;
  vv.b = opt.vb;
  mm.pack(m);
  vv.pack(v);
}

// Flat Adam over n elements with explicit bias corrections (the element
// update of net.rs:242-244).
void zlo_adam_flat(float* p, const float* g, float* m, float* v, long long n, float lr,
                   float bc1, float bc2) {
  for (long long i = 0; i < n; ++i) adam_elem(p[i], g[i], m[i], v[i], lr, 0.9f, 0.999f, bc1, bc2, 1e-8f);
}

void zlo_gae(const float* r, const float* v, const uint8_t* d, int T, float last_v, float gamma,
             float lam, float* adv, float* ret) {
  gae(r, v, d, (size_t)T, last_v, gamma, lam, adv, ret);
}

// ---------------------------------------------------------------- ActorCritic

// ActorCritic::new(.., &mut rng) where *rng_state is the Lcg's raw state
// (Lcg::new(seed) stores seed | 1); the state after construction is written
// back so the caller can keep drawing from the same stream.
void* zlo_ac_create(const int* adims, int na, const int* cdims, int nc, float init_noise_std,
                    float init_lr, uint64_t* rng_state) {
  Lcg r(1);
  r.s = *rng_state;
  void* h = new ActorCritic(
      ActorCritic::create(to_dims(adims, na), to_dims(cdims, nc), init_noise_std, init_lr, r));
  *rng_state = r.s;
  return h;
}

void zlo_ac_destroy(void* h) { delete (ActorCritic*)h; }

void zlo_ac_get(void* h, float* actor, float* critic, float* log_std, float* lr, int* t_logstd) {
  ActorCritic* ac = (ActorCritic*)h;
  if (actor) ac->actor.pack(actor);
  if (critic) ac->critic.pack(critic);
  if (log_std) std::memcpy(log_std, ac->log_std.data(), ac->log_std.size() * 4);
  if (lr) *lr = ac->lr;
  if (t_logstd) *t_logstd = ac->t_logstd;
}

// Adam moments of both nets packed like Mlp::pack, the log_std moments, and
// the three step counters (opt_actor.t, opt_critic.t, t_logstd).
void zlo_ac_get_moments(void* h, float* ma, float* va, float* mc, float* vc, float* mls,
                        float* vls, int* counters) {
  ActorCritic* ac = (ActorCritic*)h;
  auto pack = [](const Adam& a, float* m, float* v) {
    for (size_t l = 0; l < a.mw.size(); ++l) {
      if (m) {
        std::memcpy(m, a.mw[l].data(), a.mw[l].size() * 4);
        m += a.mw[l].size();
        std::memcpy(m, a.mb[l].data(), a.mb[l].size() * 4);
        m += a.mb[l].size();
      }
      if (v) {
        std::memcpy(v, a.vw[l].data(), a.vw[l].size() * 4);
        v += a.vw[l].size();
        std::memcpy(v, a.vb[l].data(), a.vb[l].size() * 4);
        v += a.vb[l].size();
      }
    }
  };
  pack(ac->opt_actor, ma, va);
  pack(ac->opt_critic, mc, vc);
  if (mls) std::memcpy(mls, ac->m_logstd.data(), ac->m_logstd.size() * 4);
  if (vls) std::memcpy(vls, ac->v_logstd.data(), ac->v_logstd.size() * 4);
  if (counters) {
    counters[0] = ac->opt_actor.t;
    counters[1] = ac->opt_critic.t;
    counters[2] = ac->t_logstd;
  }
}

void zlo_ac_set(void* h, const float* actor, const float* critic, const float* log_std,
                float lr) {
  ActorCritic* ac = (ActorCritic*)h;
  if (actor) ac->actor.unpack(actor);
  if (critic) ac->critic.unpack(critic);
  if (log_std) std::memcpy(ac->log_std.data(), log_std, ac->log_std.size() * 4);
  ac->lr = lr;
}

void zlo_ac_record_obs(void* h, const float* obs, const float* cobs) {
  ActorCritic* ac = (ActorCritic*)h;
  ac->obs_norm.update(obs);
  ac->critic_norm.update(cobs);
}

void zlo_ac_mean(void* h, const float* obs, float* out) { ((ActorCritic*)h)->mean(obs, out); }
float zlo_ac_value(void* h, const float* cobs) { return ((ActorCritic*)h)->value(cobs); }
float zlo_ac_entropy(void* h) { return ((ActorCritic*)h)->entropy(); }
float zlo_ac_logp(void* h, const float* action, const float* mean) {
  return ((ActorCritic*)h)->logp(action, mean);
}

// ActorCritic::sample with an Lcg whose state lives in *rng_state (so a
// caller can continue the same stream across calls).
float zlo_ac_sample(void* h, const float* obs, uint64_t* rng_state, float* action, float* mean) {
  Lcg r(1);
  r.s = *rng_state;
  float lp = ((ActorCritic*)h)->sample(obs, r, action, mean);
  *rng_state = r.s;
  return lp;
}

static PpoConfig to_cfg(const zlo_ppo_cfg* c) {
  PpoConfig p;
  p.gamma = c->gamma;
  p.lam = c->lam;
  p.clip = c->clip;
  p.entropy_coef = c->entropy_coef;
  p.value_coef = c->value_coef;
  p.epochs = c->epochs;
  p.minibatches = c->minibatches;
  p.max_grad_norm = c->max_grad_norm;
  p.desired_kl = c->desired_kl;
  p.lr_min = c->lr_min;
  p.lr_max = c->lr_max;
  p.adaptive_lr = c->adaptive_lr != 0;
  return p;
}

// ActorCritic::update over a structure-of-arrays batch. adv is normalised in
// place (as ppo.rs:343-348 does to the Samples). stats_out = {kl, surrogate,
// value_loss, entropy, lr}.
void zlo_ac_update(void* h, long long n, int od, int cd, const float* obs, const float* cobs,
                   const float* action, const float* mean_old, const float* logp_old,
                   const float* value_old, float* adv, const float* ret, const zlo_ppo_cfg* cfg,
                   int nthreads, int normalize_obs, float* stats_out) {
  ActorCritic* ac = (ActorCritic*)h;
  Batch b;
  b.n = (size_t)n;
  b.od = od;
  b.cd = cd;
  b.ad = ac->action_dim();
  b.obs = obs;
  b.critic_obs = cobs;
  b.action = action;
  b.mean_old = mean_old;
  b.logp_old = logp_old;
  b.value_old = value_old;
  b.adv = adv;
  b.ret = ret;
  PpoStats s = ac->update(b, to_cfg(cfg), nthreads, normalize_obs != 0);
  stats_out[0] = s.kl;
  stats_out[1] = s.surrogate;
  stats_out[2] = s.value_loss;
  stats_out[3] = s.entropy;
  stats_out[4] = s.lr;
}

// One minibatch_step over explicit sample indices (ppo.rs:388-493).
void zlo_ac_minibatch_step(void* h, long long n, int od, int cd, const float* obs,
                           const float* cobs, const float* action, const float* mean_old,
                           const float* logp_old, const float* value_old, float* adv,
                           const float* ret, const long long* idx, long long count,
                           const zlo_ppo_cfg* cfg, int nthreads, int normalize_obs,
                           float* stats_out) {
  ActorCritic* ac = (ActorCritic*)h;
  Batch b;
  b.n = (size_t)n;
  b.od = od;
  b.cd = cd;
  b.ad = ac->action_dim();
  b.obs = obs;
  b.critic_obs = cobs;
  b.action = action;
  b.mean_old = mean_old;
  b.logp_old = logp_old;
  b.value_old = value_old;
  b.adv = adv;
  b.ret = ret;
  std::vector<size_t> ix(count);
  for (long long i = 0; i < count; ++i) ix[i] = (size_t)idx[i];
  PpoStats s = ac->minibatch_step(b, ix.data(), ix.size(), to_cfg(cfg), nthreads,
                                  normalize_obs != 0);
  stats_out[0] = s.kl;
  stats_out[1] = s.surrogate;
  stats_out[2] = s.value_loss;
  stats_out[3] = s.entropy;
  stats_out[4] = s.lr;
}

// ---------------------------------------------------------- GPU-trainer mode

void* zlo_tr_create(const int* adims, int na, const int* cdims, int nc, const float* actor,
                    const float* critic, const float* log_std, float lr) {
  TrainerState* st = new TrainerState();
  st->actor = make_net(adims, na, actor);
  st->critic = make_net(cdims, nc, critic);
  size_t ad = (size_t)adims[na - 1];
  st->log_std.assign(log_std, log_std + ad);
  st->ma.assign(st->actor.num_params(), 0.0f);
  st->va.assign(st->actor.num_params(), 0.0f);
  st->mc.assign(st->critic.num_params(), 0.0f);
  st->vc.assign(st->critic.num_params(), 0.0f);
  st->mls.assign(ad, 0.0f);
  st->vls.assign(ad, 0.0f);
  st->lr = lr;
  st->gstep = 0;
  return st;
}

void zlo_tr_destroy(void* h) { delete (TrainerState*)h; }

void zlo_tr_get(void* h, float* actor, float* critic, float* log_std, float* lr,
                unsigned long long* gstep) {
  TrainerState* st = (TrainerState*)h;
  if (actor) st->actor.pack(actor);
  if (critic) st->critic.pack(critic);
  if (log_std) std::memcpy(log_std, st->log_std.data(), st->log_std.size() * 4);
  if (lr) *lr = st->lr;
  if (gstep) *gstep = st->gstep;
}

void zlo_tr_get_moments(void* h, float* ma, float* va, float* mc, float* vc, float* mls,
                        float* vls) {
  TrainerState* st = (TrainerState*)h;
  auto cp = [](float* dst, const std::vector<float>& v) {
    if (dst) std::memcpy(dst, v.data(), v.size() * 4);
  };
  cp(ma, st->ma);
  cp(va, st->va);
  cp(mc, st->mc);
  cp(vc, st->vc);
  cp(mls, st->mls);
  cp(vls, st->vls);
}

// One trainer-semantics update over already-normalised obs and already
// normalised advantages. stats_out = {kl, surrogate, value_loss, entropy, lr,
// epochs_run, last_kl}.
void zlo_tr_update(void* h, long long n, int od, int cd, const float* obs, const float* cobs,
                   const float* action, const float* mean_old, const float* logp_old,
                   const float* value_old, float* adv, const float* ret,
                   const zlo_trainer_cfg* cfg, int nthreads, float* stats_out) {
  TrainerState* st = (TrainerState*)h;
  Batch b;
  b.n = (size_t)n;
  b.od = od;
  b.cd = cd;
  b.ad = st->log_std.size();
  b.obs = obs;
  b.critic_obs = cobs;
  b.action = action;
  b.mean_old = mean_old;
  b.logp_old = logp_old;
  b.value_old = value_old;
  b.adv = adv;
  b.ret = ret;
  TrainerConfig c;
  c.clip = cfg->clip;
  c.entropy_coef = cfg->entropy_coef;
  c.value_coef = cfg->value_coef;
  c.epochs = cfg->epochs;
  c.minibatches = cfg->minibatches;
  c.grad_clip = cfg->grad_clip;
  c.desired_kl = cfg->desired_kl;
  c.lr_min = cfg->lr_min;
  c.lr_max = cfg->lr_max;
  c.adaptive_lr = cfg->adaptive_lr != 0;
  c.early_stop = cfg->early_stop != 0;
  c.clamp_after = cfg->clamp_after != 0;
  TrainerResult r = trainer_update(*st, b, c, nthreads);
  stats_out[0] = r.stats.kl;
  stats_out[1] = r.stats.surrogate;
  stats_out[2] = r.stats.value_loss;
  stats_out[3] = r.stats.entropy;
  stats_out[4] = r.stats.lr;
  stats_out[5] = (float)r.epochs_run;
  stats_out[6] = r.last_kl;
}

// Gradients of one minibatch (idx[0..count)) without clip / Adam; packed
// grads out, stats = {surrogate, value_loss, kl}.
void zlo_ppo_minibatch_grads(const int* adims, int na, const int* cdims, int nc,
                             const float* actor, const float* critic, const float* log_std,
                             long long n, const float* obs, const float* cobs,
                             const float* action, const float* mean_old, const float* logp_old,
                             const float* value_old, const float* adv, const float* ret,
                             const long long* idx, long long count, float clip,
                             float entropy_coef, float value_coef, int nthreads, float* ga_out,
                             float* gc_out, float* gls_out, float* stats) {
  Mlp a = make_net(adims, na, actor), c = make_net(cdims, nc, critic);
  size_t ad = (size_t)adims[na - 1];
  std::vector<float> ls(log_std, log_std + ad);
  Batch b;
  b.n = (size_t)n;
  b.od = adims[0];
  b.cd = cdims[0];
  b.ad = ad;
  b.obs = obs;
  b.critic_obs = cobs;
  b.action = action;
  b.mean_old = mean_old;
  b.logp_old = logp_old;
  b.value_old = value_old;
  b.adv = const_cast<float*>(adv);
  b.ret = ret;
  std::vector<size_t> ix(count);
  for (long long i = 0; i < count; ++i) ix[i] = (size_t)idx[i];
  MlpGrad ga, gc;
  std::vector<float> gls;
  minibatch_grads(a, c, ls, b, ix.data(), ix.size(), clip, entropy_coef, value_coef, nthreads, ga,
                  gc, gls, stats);
  ga.pack(ga_out);
  gc.pack(gc_out);
  std::memcpy(gls_out, gls.data(), ad * 4);
}

// ---- observation normaliser on flat state buffers float[2 * dim + 1] =
// mean[dim], m2[dim], count (the device normaliser's layout). A pending
// state with count 0 is an empty PendingNorm.

static Normalizer norm_from(const float* st, int dim) {
  Normalizer n;
  n.mean.assign(st, st + dim);
  n.m2.assign(st + dim, st + 2 * dim);
  n.count = st[2 * dim];
  return n;
}
static void norm_to(const Normalizer& n, float* st, int dim) {
  std::memcpy(st, n.mean.data(), dim * 4);
  std::memcpy(st + dim, n.m2.data(), dim * 4);
  st[2 * dim] = n.count;
}
static PendingNorm pending_from(const float* st, int dim) {
  PendingNorm p;
  p.count = st[2 * dim];
  if (p.count != 0.0f) {  // an empty PendingNorm holds no vectors
    p.mean.assign(st, st + dim);
    p.m2.assign(st + dim, st + 2 * dim);
  }
  return p;
}
static void pending_to(const PendingNorm& p, float* st, int dim) {
  for (int i = 0; i < dim; ++i) {
    st[i] = p.mean.empty() ? 0.0f : p.mean[i];
    st[dim + i] = p.m2.empty() ? 0.0f : p.m2[i];
  }
  st[2 * dim] = p.count;
}

// Normalizer::update (ppo.rs:161-168) for rows x[r * ld ..], in order.
void zlo_norm_update_rows(float* st, int dim, const float* x, int ld, long long rows) {
  Normalizer n = norm_from(st, dim);
  for (long long r = 0; r < rows; ++r) n.update(x + r * ld);
  norm_to(n, st, dim);
}

// PendingNorm::push (ppo.rs:126-137) for rows x[r * ld ..], in order.
void zlo_pending_push_rows(float* st, int dim, const float* x, int ld, long long rows) {
  PendingNorm p = pending_from(st, dim);
  for (long long r = 0; r < rows; ++r) p.push(x + r * ld, (size_t)dim);
  pending_to(p, st, dim);
}

// Normalizer::commit (ppo.rs:179-195).
void zlo_norm_commit(float* st, float* pend, int dim) {
  Normalizer n = norm_from(st, dim);
  PendingNorm p = pending_from(pend, dim);
  norm_commit(n, p);
  norm_to(n, st, dim);
  pending_to(p, pend, dim);
}

// Normalizer::normalize (ppo.rs:198-205) of each row.
void zlo_norm_normalize_rows(const float* st, int dim, const float* x, int ld, long long rows,
                             float* out, int ld_out) {
  Normalizer n = norm_from(st, dim);
  for (long long r = 0; r < rows; ++r) n.normalize(x + r * ld, out + r * ld_out);
}

// Advantage normalisation exactly as ppo.rs:343-348 / biped_train_gpu.rs:1010-1016.
void zlo_adv_normalize(float* adv, long long n) {
  float mean = 0.0f;
  for (long long i = 0; i < n; ++i) mean += adv[i];
  mean = mean / (float)n;
  float var = 0.0f;
  for (long long i = 0; i < n; ++i) var += (adv[i] - mean) * (adv[i] - mean);
  var = var / (float)n;
  float sd = std::fmax(std::sqrt(var), 1e-6f);
  for (long long i = 0; i < n; ++i) adv[i] = (adv[i] - mean) / sd;
}

}  // extern "C"
