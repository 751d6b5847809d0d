// zl_oracle.cpp — CPU restatement of zealot-rl (test infrastructure only; the
// product path never loads this). Built with -ffp-contract=off so every
// expression rounds exactly as the Rust source does.
#include "zl_oracle.hpp"

#include <algorithm>
#include <cassert>
#include <cstring>
#include <thread>

namespace zlo {

float powi_f32(float x, int n) {
  // __powisf2 (libgcc2.c / compiler-rt powisf2.c): the lowering of Rust's
  // f32::powi used by net.rs:237-238 and ppo.rs:499-500.
  unsigned int k = n < 0 ? -(unsigned int)n : (unsigned int)n;
  float y = (k % 2) ? x : 1.0f;
  while (k >>= 1) {
    x = x * x;
    if (k % 2) y = y * x;
  }
  return n < 0 ? 1.0f / y : y;
}

// ---------------------------------------------------------------- Mlp (net.rs)

Mlp Mlp::create(const std::vector<size_t>& dims, float out_scale, Lcg& rng) {
  // net.rs:61-79
  assert(dims.size() >= 2);
  Mlp net;
  net.dims = dims;
  size_t layers = dims.size() - 1;
  for (size_t l = 0; l < layers; ++l) {
    size_t fan_in = dims[l], fan_out = dims[l + 1];
    bool last = l == layers - 1;
    float s = std::sqrt(1.0f / (float)fan_in) * (last ? out_scale : 1.0f);
    std::vector<float> w(fan_out * fan_in);
    for (auto& x : w) x = rng.gauss() * s;
    net.w.push_back(std::move(w));
    net.b.push_back(std::vector<float>(fan_out, 0.0f));
  }
  return net;
}

void Mlp::forward(const float* x, std::vector<std::vector<float>>& a) const {
  // net.rs:88-108: bias-first sequential dot product, ELU on hidden layers.
  a.resize(layers() + 1);
  a[0].assign(x, x + dims[0]);
  for (size_t l = 0; l < layers(); ++l) {
    size_t fan_in = dims[l], fan_out = dims[l + 1];
    const std::vector<float>& prev = a[l];
    std::vector<float>& out = a[l + 1];
    out.assign(fan_out, 0.0f);
    bool last = l == layers() - 1;
    for (size_t o = 0; o < fan_out; ++o) {
      float z = b[l][o];
      const float* row = &w[l][o * fan_in];
      for (size_t i = 0; i < fan_in; ++i) z += row[i] * prev[i];
      out[o] = last ? z : elu(z);
    }
  }
}

void Mlp::backward(const std::vector<std::vector<float>>& a, const float* g_out, MlpGrad& g,
                   std::vector<float>* gin) const {
  // net.rs:113-140
  std::vector<float> delta(g_out, g_out + dims.back());
  for (size_t l = layers(); l-- > 0;) {
    size_t fan_in = dims[l], fan_out = dims[l + 1];
    const std::vector<float>& prev = a[l];
    const std::vector<float>& cur = a[l + 1];
    if (l != layers() - 1)
      for (size_t o = 0; o < fan_out; ++o) delta[o] *= elu_grad_from_act(cur[o]);
    std::vector<float> g_prev(fan_in, 0.0f);
    for (size_t o = 0; o < fan_out; ++o) {
      float d = delta[o];
      g.b[l][o] += d;
      const float* wrow = &w[l][o * fan_in];
      float* grow = &g.w[l][o * fan_in];
      for (size_t i = 0; i < fan_in; ++i) {
        grow[i] += d * prev[i];
        g_prev[i] += d * wrow[i];
      }
    }
    delta.swap(g_prev);
  }
  if (gin) *gin = delta;
}

size_t Mlp::num_params() const {
  size_t n = 0;
  for (size_t l = 0; l < layers(); ++l) n += w[l].size() + b[l].size();
  return n;
}

void Mlp::pack(float* out) const {
  for (size_t l = 0; l < layers(); ++l) {
    std::memcpy(out, w[l].data(), w[l].size() * 4);
    out += w[l].size();
    std::memcpy(out, b[l].data(), b[l].size() * 4);
    out += b[l].size();
  }
}

void Mlp::unpack(const float* in) {
  for (size_t l = 0; l < layers(); ++l) {
    std::memcpy(w[l].data(), in, w[l].size() * 4);
    in += w[l].size();
    std::memcpy(b[l].data(), in, b[l].size() * 4);
    in += b[l].size();
  }
}

// ------------------------------------------------------------ MlpGrad (net.rs)

MlpGrad MlpGrad::zero(const Mlp& net) {
  MlpGrad g;
  for (auto& m : net.w) g.w.push_back(std::vector<float>(m.size(), 0.0f));
  for (auto& v : net.b) g.b.push_back(std::vector<float>(v.size(), 0.0f));
  return g;
}

void MlpGrad::add(const MlpGrad& o) {  // net.rs:153-164
  for (size_t l = 0; l < w.size(); ++l)
    for (size_t i = 0; i < w[l].size(); ++i) w[l][i] += o.w[l][i];
  for (size_t l = 0; l < b.size(); ++l)
    for (size_t i = 0; i < b[l].size(); ++i) b[l][i] += o.b[l][i];
}

void MlpGrad::scale(float s) {  // net.rs:167-178
  for (auto& m : w)
    for (auto& x : m) x *= s;
  for (auto& v : b)
    for (auto& x : v) x *= s;
}

float MlpGrad::l2_norm() const {  // net.rs:181-194: one sequential f32 sum
  float s = 0.0f;
  for (auto& m : w)
    for (float x : m) s += x * x;
  for (auto& v : b)
    for (float x : v) s += x * x;
  return std::sqrt(s);
}

void MlpGrad::clip(float max_norm) {  // net.rs:197-202
  float n = l2_norm();
  if (n > max_norm && n > 0.0f) scale(max_norm / n);
}

void MlpGrad::pack(float* out) const {
  for (size_t l = 0; l < w.size(); ++l) {
    std::memcpy(out, w[l].data(), w[l].size() * 4);
    out += w[l].size();
    std::memcpy(out, b[l].data(), b[l].size() * 4);
    out += b[l].size();
  }
}

void MlpGrad::unpack(const float* in) {
  for (size_t l = 0; l < w.size(); ++l) {
    std::memcpy(w[l].data(), in, w[l].size() * 4);
    in += w[l].size();
    std::memcpy(b[l].data(), in, b[l].size() * 4);
    in += b[l].size();
  }
}

// --------------------------------------------------------------- Adam (net.rs)

Adam Adam::create(const Mlp& net) {
  Adam a;
  for (auto& m : net.w) {
    a.mw.push_back(std::vector<float>(m.size(), 0.0f));
    a.vw.push_back(std::vector<float>(m.size(), 0.0f));
  }
  for (auto& v : net.b) {
    a.mb.push_back(std::vector<float>(v.size(), 0.0f));
    a.vb.push_back(std::vector<float>(v.size(), 0.0f));
  }
  return a;
}

void Adam::step(Mlp& net, const MlpGrad& g, float lr) {  // net.rs:234-252
  t += 1;
  float bc1 = 1.0f - powi_f32(beta1, t);
  float bc2 = 1.0f - powi_f32(beta2, t);
  for (size_t l = 0; l < net.w.size(); ++l) {
    for (size_t i = 0; i < net.w[l].size(); ++i)
      adam_elem(net.w[l][i], g.w[l][i], mw[l][i], vw[l][i], lr, beta1, beta2, bc1, bc2, eps);
    for (size_t i = 0; i < net.b[l].size(); ++i)
      adam_elem(net.b[l][i], g.b[l][i], mb[l][i], vb[l][i], lr, beta1, beta2, bc1, bc2, eps);
  }
}

// --------------------------------------------------------- Normalizer (ppo.rs)

Normalizer Normalizer::create(size_t dim) {  // ppo.rs:142-148
  Normalizer n;
  n.mean.assign(dim, 0.0f);
  n.m2.assign(dim, 1.0f);
  n.count = 1.0f;
  return n;
}

void Normalizer::update(const float* x) {  // ppo.rs:161-168
  count += 1.0f;
  for (size_t i = 0; i < mean.size(); ++i) {
    float d = x[i] - mean[i];
    mean[i] += d / count;
    m2[i] += d * (x[i] - mean[i]);
  }
}

void Normalizer::normalize(const float* x, float* out) const {  // ppo.rs:198-205
  for (size_t i = 0; i < mean.size(); ++i) {
    float var = std::fmax(m2[i] / count, 1e-8f);
    float z = (x[i] - mean[i]) / std::sqrt(var);
    out[i] = z < -5.0f ? -5.0f : (z > 5.0f ? 5.0f : z);
  }
}

void PendingNorm::push(const float* x, size_t dim) {  // ppo.rs:126-137
  count += 1.0f;
  if (mean.empty()) {
    mean.assign(dim, 0.0f);
    m2.assign(dim, 0.0f);
  }
  for (size_t i = 0; i < dim; ++i) {
    float d = x[i] - mean[i];
    mean[i] += d / count;
    m2[i] += d * (x[i] - mean[i]);
  }
}

void norm_commit(Normalizer& n, PendingNorm& p) {  // ppo.rs:179-195
  if (p.count == 0.0f) return;
  float n1 = n.count, n2 = p.count, tot = n1 + n2;
  for (size_t i = 0; i < n.mean.size(); ++i) {
    float d = p.mean[i] - n.mean[i];
    n.mean[i] += d * n2 / tot;
    n.m2[i] += p.m2[i] + d * d * n1 * n2 / tot;
  }
  n.count = tot;
  p.count = 0.0f;
  p.mean.clear();
  p.m2.clear();
}

// ------------------------------------------------------- ActorCritic (ppo.rs)

ActorCritic ActorCritic::create(const std::vector<size_t>& actor_dims,
                                const std::vector<size_t>& critic_dims, float init_noise_std,
                                float init_lr, Lcg& rng) {
  // ppo.rs:235-266
  assert(critic_dims.back() == 1);
  ActorCritic ac;
  size_t ad = actor_dims.back();
  ac.actor = Mlp::create(actor_dims, 0.01f, rng);
  ac.critic = Mlp::create(critic_dims, 1.0f, rng);
  ac.opt_actor = Adam::create(ac.actor);
  ac.opt_critic = Adam::create(ac.critic);
  ac.obs_norm = Normalizer::create(actor_dims[0]);
  ac.critic_norm = Normalizer::create(critic_dims[0]);
  ac.log_std.assign(ad, std::log(init_noise_std));
  ac.m_logstd.assign(ad, 0.0f);
  ac.v_logstd.assign(ad, 0.0f);
  ac.t_logstd = 0;
  ac.lr = init_lr;
  return ac;
}

void ActorCritic::mean(const float* obs, float* out) const {
  std::vector<float> z(actor.dims[0]);
  obs_norm.normalize(obs, z.data());
  std::vector<std::vector<float>> a;
  actor.forward(z.data(), a);
  std::copy(a.back().begin(), a.back().end(), out);
}

float ActorCritic::value(const float* critic_obs) const {
  std::vector<float> z(critic.dims[0]);
  critic_norm.normalize(critic_obs, z.data());
  std::vector<std::vector<float>> a;
  critic.forward(z.data(), a);
  return a.back()[0];
}

float ActorCritic::logp(const float* action, const float* mean) const {
  float lp = 0.0f;
  for (size_t k = 0; k < action_dim(); ++k) {
    float sd = std::exp(log_std[k]);
    float d = (action[k] - mean[k]) / sd;
    lp += -0.5f * d * d - log_std[k] - kLogSqrt2Pi;
  }
  return lp;
}

float ActorCritic::entropy() const {
  float c = 0.5f + kLogSqrt2Pi;
  float s = 0.0f;
  for (float ls : log_std) s += ls + c;
  return s;
}

float ActorCritic::sample(const float* obs, Lcg& rng, float* action, float* mean_out) const {
  mean(obs, mean_out);
  for (size_t k = 0; k < action_dim(); ++k) {
    float sd = std::exp(log_std[k]);
    action[k] = mean_out[k] + sd * rng.gauss();
  }
  return logp(action, mean_out);
}

float ActorCritic::kl(const float* mean_new, const float* mean_old) const {
  float k_ = 0.0f;
  for (size_t k = 0; k < action_dim(); ++k) {
    float inv = std::exp(-log_std[k]);
    float y = (mean_new[k] - mean_old[k]) * inv;
    k_ += 0.5f * (y * y);
  }
  return k_;
}

namespace {

// ppo.rs:395 Acc = (actor grad, critic grad, log_std grad, surrogate, value_loss, kl)
struct Acc {
  MlpGrad ga, gc;
  std::vector<float> gls;
  float surr = 0, vloss = 0, kl = 0;
  // Last forward's actor means per sample (used by the trainer restatement).
};

float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

// The per-sample body of ppo.rs:408-453 (shared by both restated updates).
void fold_sample(const ActorCritic& ac, const Mlp& actor, const Mlp& critic,
                 const std::vector<float>& log_std, const Batch& batch, size_t i, float clip,
                 float entropy_coef, float value_coef, float scale, bool normalize_obs, Acc& acc,
                 std::vector<std::vector<float>>& act, std::vector<std::vector<float>>& vact,
                 std::vector<float>& zbuf, std::vector<float>& g_mean, float* mean_out) {
  size_t ad = log_std.size();
  const float* obs = batch.obs + i * batch.od;
  const float* cobs = batch.critic_obs + i * batch.cd;
  const float* action = batch.action + i * ad;
  // --- actor (normalized obs) ---
  if (normalize_obs) {
    zbuf.resize(batch.od);
    ac.obs_norm.normalize(obs, zbuf.data());
    actor.forward(zbuf.data(), act);
  } else {
    actor.forward(obs, act);
  }
  const std::vector<float>& mean = act.back();
  if (mean_out) std::copy(mean.begin(), mean.end(), mean_out);
  float lp = 0.0f;
  for (size_t k = 0; k < ad; ++k) {
    float sd = std::exp(log_std[k]);
    float d = (action[k] - mean[k]) / sd;
    lp += -0.5f * d * d - log_std[k] - kLogSqrt2Pi;
  }
  float ratio = std::exp(lp - batch.logp_old[i]);
  float a = batch.adv[i];
  float lo = 1.0f - clip, hi = 1.0f + clip;
  float surr = std::fmin(ratio * a, clampf(ratio, lo, hi) * a);
  acc.surr += surr * scale;
  bool clipped = (a >= 0.0f && ratio > hi) || (a < 0.0f && ratio < lo);
  g_mean.assign(ad, 0.0f);
  for (size_t k = 0; k < ad; ++k) {
    float inv_var = std::exp(-2.0f * log_std[k]);
    if (!clipped) {
      float d = action[k] - mean[k];
      g_mean[k] = -(a * ratio * d * inv_var) * scale;
      float dls = a * ratio * ((d * d) * inv_var - 1.0f);
      acc.gls[k] += -dls * scale;
    }
    acc.gls[k] += -entropy_coef * scale;
  }
  actor.backward(act, g_mean.data(), acc.ga, nullptr);
  // --- critic (clipped value loss, normalized obs) ---
  if (normalize_obs) {
    zbuf.resize(batch.cd);
    ac.critic_norm.normalize(cobs, zbuf.data());
    critic.forward(zbuf.data(), vact);
  } else {
    critic.forward(cobs, vact);
  }
  float v = vact.back()[0];
  float vo = batch.value_old[i], r = batch.ret[i];
  float v_clipped = vo + clampf(v - vo, -clip, clip);
  float l_unclipped = (v - r) * (v - r);
  float l_clipped = (v_clipped - r) * (v_clipped - r);
  float vloss, dv;
  if (l_clipped > l_unclipped) {
    vloss = l_clipped;
    dv = 2.0f * (v_clipped - r);
  } else {
    vloss = l_unclipped;
    dv = 2.0f * (v - r);
  }
  acc.vloss += vloss * scale;
  float gv = value_coef * dv * scale;
  critic.backward(vact, &gv, acc.gc, nullptr);
  // ActorCritic::kl (ppo.rs:327-334) with the live log_std.
  float klv = 0.0f;
  for (size_t k = 0; k < ad; ++k) {
    float inv = std::exp(-log_std[k]);
    float y = (mean[k] - batch.mean_old[i * ad + k]) * inv;
    klv += 0.5f * (y * y);
  }
  acc.kl += klv * scale;
}

// Fold `count` samples (indices idx[0..count)) over nthreads contiguous chunks,
// then reduce the per-thread accumulators left to right (ppo.rs:406-462).
Acc fold_minibatch(const ActorCritic& ac, const Mlp& actor, const Mlp& critic,
                   const std::vector<float>& log_std, const Batch& batch, const size_t* idx,
                   size_t count, float clip, float entropy_coef, float value_coef,
                   bool normalize_obs, int nthreads, float* means_out) {
  float scale = 1.0f / (float)count;
  size_t ad = log_std.size();
  if (nthreads < 1) nthreads = 1;
  if ((size_t)nthreads > count) nthreads = (int)std::max<size_t>(count, 1);
  std::vector<Acc> accs(nthreads);
  for (auto& a : accs) {
    a.ga = MlpGrad::zero(actor);
    a.gc = MlpGrad::zero(critic);
    a.gls.assign(ad, 0.0f);
  }
  auto work = [&](int t) {
    size_t lo = count * t / nthreads, hi = count * (t + 1) / nthreads;
    std::vector<std::vector<float>> act, vact;
    std::vector<float> zbuf, g_mean;
    for (size_t j = lo; j < hi; ++j)
      fold_sample(ac, actor, critic, log_std, batch, idx[j], clip, entropy_coef, value_coef,
                  scale, normalize_obs, accs[t], act, vact, zbuf, g_mean,
                  means_out ? means_out + j * ad : nullptr);
  };
  if (nthreads == 1) {
    work(0);
  } else {
    std::vector<std::thread> th;
    for (int t = 0; t < nthreads; ++t) th.emplace_back(work, t);
    for (auto& x : th) x.join();
  }
  Acc out = std::move(accs[0]);
  for (int t = 1; t < nthreads; ++t) {
    out.ga.add(accs[t].ga);
    out.gc.add(accs[t].gc);
    for (size_t k = 0; k < ad; ++k) out.gls[k] += accs[t].gls[k];
    out.surr = out.surr + accs[t].surr;
    out.vloss = out.vloss + accs[t].vloss;
    out.kl = out.kl + accs[t].kl;
  }
  return out;
}

}  // namespace

PpoStats ActorCritic::minibatch_step(const Batch& batch, const size_t* idx, size_t count,
                                     const PpoConfig& cfg, int nthreads, bool normalize_obs) {
  // ppo.rs:388-493
  Acc acc = fold_minibatch(*this, actor, critic, log_std, batch, idx, count, cfg.clip,
                           cfg.entropy_coef, cfg.value_coef, normalize_obs, nthreads, nullptr);
  PpoStats st;
  st.surrogate = acc.surr;
  st.value_loss = acc.vloss;
  st.kl = acc.kl;
  st.entropy = entropy();
  if (cfg.adaptive_lr) {
    if (st.kl > cfg.desired_kl * 2.0f)
      lr = std::fmax(lr / 1.5f, cfg.lr_min);
    else if (st.kl > 0.0f && st.kl < cfg.desired_kl / 2.0f)
      lr = std::fmin(lr * 1.5f, cfg.lr_max);
  }
  acc.ga.clip(cfg.max_grad_norm);
  acc.gc.clip(cfg.max_grad_norm);
  opt_actor.step(actor, acc.ga, lr);
  opt_critic.step(critic, acc.gc, lr);
  step_log_std(acc.gls.data());
  st.lr = lr;
  return st;
}

void ActorCritic::step_log_std(const float* g) {  // ppo.rs:496-510
  t_logstd += 1;
  const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
  float bc1 = 1.0f - powi_f32(b1, t_logstd);
  float bc2 = 1.0f - powi_f32(b2, t_logstd);
  for (size_t k = 0; k < action_dim(); ++k) {
    m_logstd[k] = b1 * m_logstd[k] + (1.0f - b1) * g[k];
    v_logstd[k] = b2 * v_logstd[k] + (1.0f - b2) * g[k] * g[k];
    float step = lr * (m_logstd[k] / bc1) / (std::sqrt(v_logstd[k] / bc2) + eps);
    log_std[k] = clampf(log_std[k] - step, -1.6f, 1.0f);
  }
}

PpoStats ActorCritic::update(Batch& batch, const PpoConfig& cfg, int nthreads,
                             bool normalize_obs) {
  // ppo.rs:338-384
  size_t n = batch.n;
  assert(n >= (size_t)cfg.minibatches);
  float mean = 0.0f;
  for (size_t i = 0; i < n; ++i) mean += batch.adv[i];
  mean = mean / (float)n;
  float var = 0.0f;
  for (size_t i = 0; i < n; ++i) var += (batch.adv[i] - mean) * (batch.adv[i] - mean);
  var = var / (float)n;
  float sd = std::fmax(std::sqrt(var), 1e-6f);
  for (size_t i = 0; i < n; ++i) batch.adv[i] = (batch.adv[i] - mean) / sd;

  size_t mb = n / cfg.minibatches;
  PpoStats stats;
  stats.lr = lr;
  std::vector<size_t> order(n);
  for (int e = 0; e < cfg.epochs; ++e) {
    for (size_t i = 0; i < n; ++i) order[i] = i;
    Lcg sh((uint64_t)t_logstd + 1);
    for (size_t i = n - 1; i >= 1; --i) {
      size_t j = (size_t)(sh.unit() * (float)(i + 1));
      std::swap(order[i], order[std::min(j, i)]);
    }
    PpoStats ep;
    for (int m = 0; m < cfg.minibatches; ++m) {
      PpoStats s = minibatch_step(batch, &order[m * mb], mb, cfg, nthreads, normalize_obs);
      ep.kl += s.kl;
      ep.surrogate += s.surrogate;
      ep.value_loss += s.value_loss;
      ep.entropy += s.entropy;
    }
    float inv = 1.0f / (float)cfg.minibatches;
    stats.kl = ep.kl * inv;
    stats.surrogate = ep.surrogate * inv;
    stats.value_loss = ep.value_loss * inv;
    stats.entropy = ep.entropy * inv;
    stats.lr = lr;
  }
  return stats;
}

void gae(const float* rewards, const float* values, const uint8_t* dones, size_t t,
         float last_value, float gamma, float lam, float* adv, float* ret) {
  // ppo.rs:681-703
  float acc = 0.0f;
  float next_v = last_value;
  for (size_t i = t; i-- > 0;) {
    float nt = dones[i] ? 0.0f : 1.0f;
    float delta = rewards[i] + gamma * next_v * nt - values[i];
    acc = delta + gamma * lam * nt * acc;
    adv[i] = acc;
    ret[i] = acc + values[i];
    next_v = values[i];
  }
}

void minibatch_grads(const Mlp& actor, const Mlp& critic, const std::vector<float>& log_std,
                     const Batch& batch, const size_t* idx, size_t count, float clip,
                     float entropy_coef, float value_coef, int nthreads, MlpGrad& ga, MlpGrad& gc,
                     std::vector<float>& gls, float stats[3]) {
  ActorCritic dummy;
  Acc acc = fold_minibatch(dummy, actor, critic, log_std, batch, idx, count, clip, entropy_coef,
                           value_coef, false, nthreads, nullptr);
  ga = std::move(acc.ga);
  gc = std::move(acc.gc);
  gls = std::move(acc.gls);
  stats[0] = acc.surr;
  stats[1] = acc.vloss;
  stats[2] = acc.kl;
}

// ------------------------------------------------------------ GPU-trainer mode

TrainerResult trainer_update(TrainerState& st, const Batch& batch, const TrainerConfig& cfg,
                             int nthreads) {
  // src/bin/biped_train_gpu.rs:1004-1553 (after advantage normalisation).
  size_t total = batch.n;
  size_t mb = total / cfg.minibatches;
  size_t n_mb = total / mb;
  size_t ad = st.log_std.size();
  std::vector<float> log_std_old = st.log_std;  // :1115
  ActorCritic dummy;                             // normalisers unused (obs pre-normalised)
  std::vector<size_t> idx(mb);
  std::vector<float> means_last(mb * ad);
  TrainerResult res;
  const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
  size_t na = st.actor.num_params(), nc = st.critic.num_params();
  std::vector<float> pa(na), pc(nc), ga(na), gc(nc);
  for (int e = 0; e < cfg.epochs; ++e) {
    st.gstep += n_mb;  // :1165-1167
    int tt = (int)std::min<uint64_t>(st.gstep, 1ULL << 30);
    float bc1 = 1.0f - powi_f32(0.9f, tt);
    float bc2 = 1.0f - powi_f32(0.999f, tt);
    PpoStats ep;
    for (size_t k = 0; k < n_mb; ++k) {
      for (size_t c = 0; c < mb; ++c) idx[c] = k * mb + c;  // contiguous columns :1185-1250
      bool last = k == n_mb - 1;
      Acc acc = fold_minibatch(dummy, st.actor, st.critic, st.log_std, batch, idx.data(), mb,
                               cfg.clip, cfg.entropy_coef, cfg.value_coef, false, nthreads,
                               last ? means_last.data() : nullptr);
      ep.surrogate += acc.surr;
      ep.value_loss += acc.vloss;
      ep.kl += acc.kl;
      float ent = 0.0f;
      for (float ls : st.log_std) ent += ls + (0.5f + kLogSqrt2Pi);
      ep.entropy += ent;
      // Global clip over actor dw, actor db, critic dw, critic db, dls (:1368-1452):
      // one f32 sum of squares per tensor, summed over slots in that order.
      if (cfg.grad_clip > 0.0f) {
        float total_sq = 0.0f;
        auto sq = [](const std::vector<float>& v) {
          float s = 0.0f;
          for (float x : v) s += x * x;
          return s;
        };
        for (const MlpGrad* g : {&acc.ga, &acc.gc}) {
          for (auto& m : g->w) total_sq += sq(m);
          for (auto& v : g->b) total_sq += sq(v);
        }
        total_sq += sq(acc.gls);
        float norm = std::sqrt(total_sq);
        if (norm > cfg.grad_clip) {
          float sc = cfg.grad_clip / norm;
          acc.ga.scale(sc);
          acc.gc.scale(sc);
          for (auto& x : acc.gls) x *= sc;
        }
      }
      // Adam with the epoch's shared (lr, bc1, bc2) (:1453-1461).
      st.actor.pack(pa.data());
      acc.ga.pack(ga.data());
      for (size_t i = 0; i < na; ++i)
        adam_elem(pa[i], ga[i], st.ma[i], st.va[i], st.lr, b1, b2, bc1, bc2, eps);
      st.actor.unpack(pa.data());
      st.critic.pack(pc.data());
      acc.gc.pack(gc.data());
      for (size_t i = 0; i < nc; ++i)
        adam_elem(pc[i], gc[i], st.mc[i], st.vc[i], st.lr, b1, b2, bc1, bc2, eps);
      st.critic.unpack(pc.data());
      for (size_t i = 0; i < ad; ++i)
        adam_elem(st.log_std[i], acc.gls[i], st.mls[i], st.vls[i], st.lr, b1, b2, bc1, bc2, eps);
    }
    float inv = 1.0f / (float)n_mb;
    res.stats.surrogate = ep.surrogate * inv;
    res.stats.value_loss = ep.value_loss * inv;
    res.stats.kl = ep.kl * inv;
    res.stats.entropy = ep.entropy * inv;
    res.epochs_run = e + 1;
    // Per-epoch full-Gaussian KL on the last minibatch (:1469-1492).
    size_t last_off = (n_mb - 1) * mb;
    float kl = 0.0f;
    for (size_t c = 0; c < mb; ++c) {
      for (size_t k = 0; k < ad; ++k) {
        float ls_new = st.log_std[k], ls_old = log_std_old[k];
        float sig_old2 = std::exp(2.0f * ls_old);
        float inv_sig_new2 = std::exp(-2.0f * ls_new);
        float dmu = means_last[c * ad + k] - batch.mean_old[(last_off + c) * ad + k];
        kl += (ls_new - ls_old) + 0.5f * (sig_old2 + dmu * dmu) * inv_sig_new2 - 0.5f;
      }
    }
    kl /= (float)mb;
    res.last_kl = kl;
    if (cfg.adaptive_lr) {  // :1497-1501
      if (kl > cfg.desired_kl * 2.0f)
        st.lr = std::fmax(st.lr / 1.5f, cfg.lr_min);
      else if (kl > 0.0f && kl < cfg.desired_kl / 2.0f)
        st.lr = std::fmin(st.lr * 1.5f, cfg.lr_max);
    }
    if (cfg.early_stop && kl > cfg.desired_kl * 5.0f) break;  // :1513-1515
  }
  if (cfg.clamp_after)  // :1529-1541
    for (auto& v : st.log_std) v = clampf(v, -1.6f, 0.0f);
  res.stats.lr = st.lr;
  return res;
}

}  // namespace zlo
