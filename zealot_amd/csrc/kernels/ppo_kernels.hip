// ppo_kernels.hip — the non-GEMM kernels of the PPO update on gfx950.
//
// All are bandwidth/latency-bound and written as single-pass, coalesced
// kernels with deterministic (fixed-order, atomic-free) reductions. FP
// contraction is off for the whole code object, so every expression rounds
// like the reference's Rust source (zealot-rl/src/net.rs, ppo.rs).
#pragma once
#include "common.hip"
#include "gemm_mfma.hip"  // reduce_all_body (zk_reduce_all is defined here, with its tail block)

namespace zk {

// ------------------------------------------------------------------ losses

// Sum of v over lanes base .. base+n-1 of the wavefront (n <= G), added left
// to right like the reference's serial loops over action components; every
// lane gets the result. The log-probabilities reach a few hundred in
// magnitude, where a different summation order moves the PPO ratio by ~1e-5
// relative, so the order is kept. The lane reads are independent, so they
// are issued 16 at a time ahead of their adds (one shuffle latency per 16
// components, 16 registers).
template <int G>
__device__ __forceinline__ float lanes_sum_ordered(float v, int base, int n) {
  constexpr int kBatch = 16;
  float s = 0.f;
#pragma unroll
  for (int j0 = 0; j0 < G; j0 += kBatch) {
    float t[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) t[j] = __shfl(v, base + j0 + j, 64);
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (j0 + j < n) s += t[j];
  }
  return s;
}

// Per-sample body of zealot-rl/src/ppo.rs:411-432 and :452 (actor half of
// minibatch_step). One lane group per sample with lane k holding action
// component k, so a sample's mean / action / gradient rows are read and
// written as contiguous runs; the sums over components (logp, KL) run over
// the group's lanes in component order. Each lane accumulates its
// component's log_std gradient over the samples its group visits (in order),
// and the groups of a block are then combined in a fixed order:
// deterministic per-block partials (the rayon fold of :406-462 has no fixed
// order either).
template <int G>
__device__ void actor_loss_body(const ActorLossArgs& p) {
  constexpr int kMaxGroups = kLossThreads / 32;
  __shared__ float sh_g[kMaxGroups][64];
  __shared__ float sh_s[kMaxGroups][2];
  if (p.guard && *p.guard == 0) return;
  const int t = threadIdx.x;
  const int ng = kLossThreads / G;
  const int grp = t / G, k = t % G;
  const int base = (t & 63) - k;  // first lane of this group in the wavefront
  const int A = p.A;
  const bool on = k < A;
  const float ls = on ? p.log_std[k] : 0.f;
  const float sd = expf(ls);
  const float inv_var = expf(-2.0f * ls);
  const float inv_sd = expf(-ls);
  const float lo = 1.0f - p.clip, hi = 1.0f + p.clip;
  float gacc = 0.f, sacc = 0.f, kacc = 0.f;
  const int r0 = blockIdx.x * p.rows_per_block;
  const int r1 = min(p.rows, r0 + p.rows_per_block);
  // A group's rows are taken R at a time with all their loads issued before
  // the first row is computed (one memory latency per R rows).
  struct In {
    float mu, act, lpo, adv, mo;
  };
  auto fetch = [&](int rr) {
    In x;
    const long long s = p.perm ? p.perm[p.row0 + rr] : (long long)(p.row0 + rr);
    x.mu = on ? p.mean[(long long)rr * p.ldm + (long long)k * p.cm] : 0.f;
    x.act = on ? p.action[s * p.ldact + (long long)k * p.cact] : 0.f;
    x.lpo = p.logp_old[s];
    x.adv = p.adv[s];
    x.mo = (p.mean_old && on) ? p.mean_old[s * p.ldmo + (long long)k * p.cmo] : 0.f;
    return x;
  };
  // Rows per group whose loads are issued together (two for 64-lane groups,
  // whose ordered sums already hold 64 shuffled values in registers).
  constexpr int R = G == 32 ? 4 : 2;
  for (int rb = r0 + grp; rb < r1; rb += ng * R) {
    In in[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int r = rb + j * ng;
      in[j] = r < r1 ? fetch(r) : In{};
    }
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int r = rb + j * ng;
      if (r >= r1) break;
      const In& cur = in[j];
      const float mu = cur.mu, act = cur.act;
      // ActorCritic::logp, ppo.rs:297-305
      const float dz = (act - mu) / sd;
      const float lp = lanes_sum_ordered<G>(on ? -0.5f * dz * dz - ls - kLogSqrt2Pi : 0.f, base, A);
      const float ratio = expf(lp - cur.lpo);
      const float a = cur.adv;
      const float surr = fminf(ratio * a, clampf(ratio, lo, hi) * a);
      const bool clipped = (a >= 0.0f && ratio > hi) || (a < 0.0f && ratio < lo);
      float gm = 0.f, c = 0.f;
      if (!clipped) {
        const float d = act - mu;
        gm = -(a * ratio * d * inv_var) * p.scale;
        const float dls = a * ratio * ((d * d) * inv_var - 1.0f);
        c = -dls * p.scale;
      }
      c += -p.entropy_coef * p.scale;
      if (on) {
        p.delta[(long long)r * p.ldd + (long long)k * p.cdd] = gm;
        gacc += c;
      }
      sacc += surr * p.scale;
      if (p.mean_old) {  // ActorCritic::kl, ppo.rs:327-334
        const float y = (mu - cur.mo) * inv_sd;
        kacc += lanes_sum_ordered<G>(on ? 0.5f * (y * y) : 0.f, base, A) * p.scale;
      }
    }
  }
  sh_g[grp][k] = gacc;
  if (k == 0) {
    sh_s[grp][0] = sacc;
    sh_s[grp][1] = kacc;
  }
  __syncthreads();
  // Partials component-major ([A][blocks], [2][blocks]) so that each
  // quantity's partials are contiguous for the reductions that follow.
  if (t < A) {
    float g = 0.f;
    for (int j = 0; j < ng; ++j) g += sh_g[j][t];
    p.gls_part[(long long)t * gridDim.x + blockIdx.x] = g;
  } else if (t == 64 || t == 65) {
    const int q = t - 64;
    float v = 0.f;
    for (int j = 0; j < ng; ++j) v += sh_s[j][q];
    p.stat_part[(long long)q * gridDim.x + blockIdx.x] = v;
  }
}

// zealot-rl/src/ppo.rs:436-450 (clipped value loss; the clamp's derivative is
// ignored, so the gradient flows through v_clipped as if it were v).
__device__ void value_loss_body(const ValueLossArgs& p) {
  __shared__ float red[kThreads];
  if (p.guard && *p.guard == 0) return;
  const int t = threadIdx.x;
  const int r = blockIdx.x * kThreads + t;
  float vl_c = 0.f;
  if (r < p.rows) {
    const long long s = p.perm ? p.perm[p.row0 + r] : (long long)(p.row0 + r);
    const float v = p.v[(long long)r * p.ldv];
    const float vo = p.value_old[s], R = p.ret[s];
    const float vc = vo + clampf(v - vo, -p.clip, p.clip);
    const float lu = (v - R) * (v - R);
    const float lc = (vc - R) * (vc - R);
    float vloss, dv;
    if (lc > lu) {
      vloss = lc;
      dv = 2.0f * (vc - R);
    } else {
      vloss = lu;
      dv = 2.0f * (v - R);
    }
    vl_c = vloss * p.scale;
    p.delta[(long long)r * p.ldd] = p.value_coef * dv * p.scale;
  }
  const float tot = block_sum(vl_c, red);
  if (t == 0) p.stat_part[blockIdx.x] = tot;
}

// ------------------------------------------------- grad norm / finalize / Adam

// Per-block sum of squares over fixed chunks of two contiguous ranges.
__device__ void sumsq_body(const SumsqArgs& p) {
  __shared__ float red[kThreads];
  if (p.guard && *p.guard == 0) return;
  const int b = blockIdx.x;
  long long off, len;
  int cb;
  if (b < p.blocks0) {
    off = p.off0;
    len = p.len0;
    cb = b;
  } else {
    off = p.off1;
    len = p.len1;
    cb = b - p.blocks0;
  }
  const long long lo = (long long)cb * p.chunk;
  const long long hi = min(len, lo + p.chunk);
  const float* x = p.x + off;
  float s = 0.f;
  if ((p.chunk & 3) == 0 && ((uintptr_t)x & 15u) == 0) {
    // Quads (lo is a multiple of 4), then the scalar tail of the last chunk.
    const long long hi4 = lo + ((hi - lo) & ~3LL);
    for (long long i = lo + 4 * threadIdx.x; i < hi4; i += 4 * kThreads) {
      const float4 v = *reinterpret_cast<const float4*>(x + i);
      s += v.x * v.x;
      s += v.y * v.y;
      s += v.z * v.z;
      s += v.w * v.w;
    }
    for (long long i = hi4 + threadIdx.x; i < hi; i += kThreads) s += x[i] * x[i];
  } else {
    for (long long i = lo + threadIdx.x; i < hi; i += kThreads) {
      const float v = x[i];
      s += v * v;
    }
  }
  const float tot = block_sum(s, red);
  if (threadIdx.x == 0) p.part[b] = tot;
}

// Scalar tail of one minibatch step, the part that needs only the loss
// partials: ppo.rs:464-489 (ActorCritic::update semantics) or
// src/bin/biped_train_gpu.rs:1350-1452 (trainer semantics), every scalar kept
// on the device. Runs as the extra last block of zk_reduce_all (the loss
// partials are complete when that launch starts); the clip scales follow in
// zk_adam, which also needs this block's log_std squared norm (sq_part[nsq]).
__device__ void minibatch_tail_body(const FinalizeArgs& p) {
  // Quantities 0..2: surrogate, kl, value loss; 3..3+A-1: the log_std
  // gradient, each a sum over per-block partials. A group of 32 lanes takes
  // quantities g, g + 32, ...: lane l adds partials l, l + 32, ... in order
  // (loads issued 8 at a time), then the group's lanes are combined by a
  // fixed butterfly, so the result is deterministic.
  constexpr int kMaxA = 256;
  constexpr int kQ = 3;
  __shared__ float q[kQ + kMaxA];
  const int t = threadIdx.x;
  const int wave = t >> 6, lane = t & 63;
  const int A = p.pp.A;
  const int nq = kQ + A;
  const int grp = t >> 5, gln = t & 31;
  constexpr int kGroups = kReduceAllThreads / 32;
  for (int j = grp; j < nq; j += kGroups) {
    const float* ptr;
    int n;
    if (j == 0) {
      ptr = p.astat_part, n = p.nb_a;
    } else if (j == 1) {
      ptr = p.astat_part + p.nb_a, n = p.nb_a;
    } else if (j == 2) {
      ptr = p.vstat_part, n = p.nb_v;
    } else {
      ptr = p.gls_part + (long long)(j - kQ) * p.nb_a, n = p.nb_a;
    }
    float v = 0.f;
    for (int i0 = gln; i0 < n; i0 += 8 * 32) {
      float tv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) tv[u] = i0 + 32 * u < n ? ptr[i0 + 32 * u] : 0.f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (i0 + 32 * u < n) v += tv[u];
    }
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) v = v + __shfl_xor(v, m, 32);
    if (gln == 0) {
      q[j] = v;
      if (j >= kQ) p.g_logstd[j - kQ] = v;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  // Squared norm of the log_std gradient and the entropy
  // (ActorCritic::entropy, ppo.rs:308-311, pre-step log_std), lane-strided.
  const float c = 0.5f + kLogSqrt2Pi;
  float gl = 0.f, el = 0.f;
  for (int k = lane; k < A; k += 64) {
    const float g = q[kQ + k];
    gl += g * g;
    el += p.log_std[k] + c;
  }
  const float sq_l = wave_sum(gl);
  const float ent = wave_sum(el);
  if (lane != 0) return;
  DevState* st = p.st;
  const PpoParams& pp = p.pp;
  const float surr = q[0], kl = q[1], vloss = q[2];
  p.sq_part[p.nsq] = sq_l;
  if (pp.mode == 0) {
    if (pp.adaptive_lr) {  // ppo.rs:476-482
      if (kl > pp.desired_kl * 2.0f)
        st->lr = fmaxf(st->lr / 1.5f, pp.lr_min);
      else if (kl > 0.0f && kl < pp.desired_kl / 2.0f)
        st->lr = fminf(st->lr * 1.5f, pp.lr_max);
    }
    st->norm[2] = sqrtf(sq_l);
    st->t += 1;  // Adam::step / step_log_std advance together (net.rs:235, ppo.rs:497)
    st->bc1 = 1.0f - powi_f32(pp.beta1, st->t);
    st->bc2 = 1.0f - powi_f32(pp.beta2, st->t);
  }
  st->ep_kl += kl;
  st->ep_surr += surr;
  st->ep_vloss += vloss;
  st->ep_ent += ent;
  st->mb_in_epoch += 1;
}

// The clip scales of one minibatch step from zk_reduce_all's squared-norm
// partials (AdamArgs::clip): MlpGrad::clip per net (net.rs:197-202; log_std
// is not clipped) or the trainer's global clip over actor + critic + log_std
// (src/bin/biped_train_gpu.rs:1368-1452). Every block of zk_adam sums the
// partials in the same fixed order (thread-strided, then a fixed tree), so
// all blocks use the same scales; block 0 records them and the norms in st.
__device__ __forceinline__ void adam_clip_scales(const AdamArgs& p, float* s0, float* s1, float* s2) {
  __shared__ float red[kThreads];
  float a = 0.f, c = 0.f;
  for (int i = threadIdx.x; i < p.nsq; i += kThreads) {
    if (i < p.nsq_a)
      a += p.sq_part[i];
    else
      c += p.sq_part[i];
  }
  const float sq_a = block_sum<kThreads>(a, red);
  const float sq_c = block_sum<kThreads>(c, red);
  const float mg = p.max_grad_norm;
  const bool rec = blockIdx.x == 0 && threadIdx.x == 0;
  if (p.clip == 1) {
    const float na = sqrtf(sq_a), nc = sqrtf(sq_c);
    *s0 = (na > mg && na > 0.0f) ? mg / na : 1.0f;
    *s1 = (nc > mg && nc > 0.0f) ? mg / nc : 1.0f;
    *s2 = 1.0f;
    if (rec) {
      p.st->norm[0] = na;
      p.st->norm[1] = nc;
    }
  } else {
    float sc = 1.0f;
    if (mg > 0.0f) {
      const float norm = sqrtf(sq_a + sq_c + p.sq_part[p.nsq]);
      if (norm > mg) sc = mg / norm;
      if (rec) p.st->norm[0] = norm;
    }
    *s0 = *s1 = *s2 = sc;
  }
  if (rec) {
    p.st->scale[0] = *s0;
    p.st->scale[1] = *s1;
    p.st->scale[2] = *s2;
  }
}

// Adam element update of zealot-rl/src/net.rs:240-245 over one flat buffer
// holding every tensor of the update, float4-vectorised.
__device__ void adam_body(const AdamArgs& p) {
  if (p.guard && *p.guard == 0) return;
  // The element loads go first: they do not depend on the clip scales, so
  // they are in flight while the block takes the scales.
  const long long i0 = ((long long)blockIdx.x * kThreads + threadIdx.x) * 4;
  const bool quad = i0 + 4 <= p.n &&
                    ((((uintptr_t)p.p | (uintptr_t)p.g | (uintptr_t)p.m | (uintptr_t)p.v) & 15u) == 0);
  float x[4], g[4], m[4], v[4];
  if (quad) {
    const float4 x4 = *reinterpret_cast<const float4*>(p.p + i0);
    const float4 g4 = *reinterpret_cast<const float4*>(p.g + i0);
    const float4 m4 = *reinterpret_cast<const float4*>(p.m + i0);
    const float4 v4 = *reinterpret_cast<const float4*>(p.v + i0);
    x[0] = x4.x, x[1] = x4.y, x[2] = x4.z, x[3] = x4.w;
    g[0] = g4.x, g[1] = g4.y, g[2] = g4.z, g[3] = g4.w;
    m[0] = m4.x, m[1] = m4.y, m[2] = m4.z, m[3] = m4.w;
    v[0] = v4.x, v[1] = v4.y, v[2] = v4.z, v[3] = v4.w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = i0 + j < p.n;
      x[j] = in ? p.p[i0 + j] : 0.f;
      g[j] = in ? p.g[i0 + j] : 0.f;
      m[j] = in ? p.m[i0 + j] : 0.f;
      v[j] = in ? p.v[i0 + j] : 0.f;
    }
  }
  float lr = p.lr, bc1 = p.bc1, bc2 = p.bc2;
  float s0 = 1.f, s1 = 1.f, s2 = 1.f;
  if (p.st) {
    lr = p.st->lr;
    bc1 = p.st->bc1;
    bc2 = p.st->bc2;
    if (p.clip) {
      adam_clip_scales(p, &s0, &s1, &s2);  // every thread of the block takes part
    } else {
      s0 = p.st->scale[0];
      s1 = p.st->scale[1];
      s2 = p.st->scale[2];
    }
  }
  if (i0 >= p.n) return;
  const float b1 = p.beta1, b2 = p.beta2, eps = p.eps;
  const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const long long i = i0 + j;
    const int grp = i < p.end_a ? 0 : (i < p.end_c ? 1 : 2);
    const float sc = grp == 0 ? s0 : (grp == 1 ? s1 : s2);
    const float gr = g[j] * sc;
    m[j] = b1 * m[j] + omb1 * gr;
    v[j] = b2 * v[j] + omb2 * gr * gr;
    float xn = x[j] - lr * (m[j] / bc1) / (sqrtf(v[j] / bc2) + eps);
    if (grp == 2 && p.clamp_ls) xn = clampf(xn, -1.6f, 1.0f);
    x[j] = xn;
  }
  if (quad) {
    *reinterpret_cast<float4*>(p.m + i0) = make_float4(m[0], m[1], m[2], m[3]);
    *reinterpret_cast<float4*>(p.v + i0) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p.p + i0) = make_float4(x[0], x[1], x[2], x[3]);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (i0 + j < p.n) {
        p.m[i0 + j] = m[j];
        p.v[i0 + j] = v[j];
        p.p[i0 + j] = x[j];
      }
    }
  }
}

// --------------------------------------------------------------- epoch logic

// Opening of an epoch (zk_epoch_begin, or the tail of zk_epoch_end for the
// next one): the trainer's gstep advance and bias corrections, and cleared
// epoch sums.
__device__ __forceinline__ void open_epoch(DevState* st, const PpoParams& pp) {
  if (pp.mode == 1) {  // biped_train_gpu.rs:1165-1167
    st->gstep += (unsigned long long)pp.n_mb;
    const unsigned long long cap = 1ull << 30;
    const int tt = (int)(st->gstep < cap ? st->gstep : cap);
    st->bc1 = 1.0f - powi_f32(pp.beta1, tt);
    st->bc2 = 1.0f - powi_f32(pp.beta2, tt);
  }
  st->ep_kl = 0.f;
  st->ep_surr = 0.f;
  st->ep_vloss = 0.f;
  st->ep_ent = 0.f;
  st->mb_in_epoch = 0;
}

__device__ void epoch_begin_body(const EpochBeginArgs& p) {
  if (p.guard && *p.guard == 0) return;
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  open_epoch(p.st, p.pp);
}

// Full-Gaussian KL(old || new) of src/bin/biped_train_gpu.rs:1478-1491, one
// thread per row of the last minibatch, block partials.
__device__ void kl_body(const KlArgs& p) {
  __shared__ float red[kThreads];
  if (p.guard && *p.guard == 0) return;
  const int r = blockIdx.x * kThreads + threadIdx.x;
  float acc = 0.f;
  if (r < p.rows) {
    const long long s = p.perm ? p.perm[p.row0 + r] : (long long)(p.row0 + r);
    for (int k = 0; k < p.A; ++k) {
      const float ls_new = p.log_std[k], ls_old = p.log_std_old[k];
      const float sig_old2 = expf(2.0f * ls_old);
      const float inv_sig_new2 = expf(-2.0f * ls_new);
      const float dmu = p.mean[(long long)r * p.ldm + k] - p.mean_old[s * p.ldmo + k];
      acc += (ls_new - ls_old) + 0.5f * (sig_old2 + dmu * dmu) * inv_sig_new2 - 0.5f;
    }
  }
  const float tot = block_sum(acc, red);
  if (threadIdx.x == 0) p.part[blockIdx.x] = tot;
}

// End of an epoch (one block of kFinalizeThreads): epoch statistics, and in
// trainer mode the full-Gaussian KL of the last minibatch
// (biped_train_gpu.rs:1478-1491), the adaptive learning rate and the early
// stop. From zk_head's per-component sums S_k = sum_r (mu_rk - mu_old_rk)^2
// (kl_form 1) the mean over the R rows of
//   sum_k log(sig_new/sig_old) + (sig_old^2 + dmu^2) / (2 sig_new^2) - 1/2
// is sum_k c_k + S_k / (2 R sig_new_k^2) with
//   c_k = d - 1/2 + exp(-2 d) / 2 = (expm1(-2 d) + 2 d) / 2,  d = ls_new - ls_old,
// the same quantity with the per-row constant computed once (and without
// cancellation) per component.
__device__ void epoch_end_body(const EpochEndArgs& p) {
  constexpr int kMaxA = 256;
  __shared__ float sk[kMaxA];
  if (*p.active == 0) return;
  const int t = threadIdx.x;
  const PpoParams& pp = p.pp;
  const bool kl_on = pp.mode == 1 && p.kl_part != nullptr;
  if (kl_on && p.kl_form == 1) {
    const int grp = t >> 5, gln = t & 31;
    for (int k = grp; k < pp.A; k += kFinalizeThreads / 32) {
      const float* ptr = p.kl_part + (long long)k * p.nkl;
      float v = 0.f;
      for (int i0 = gln; i0 < p.nkl; i0 += 8 * 32) {
        float tv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) tv[u] = i0 + 32 * u < p.nkl ? ptr[i0 + 32 * u] : 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (i0 + 32 * u < p.nkl) v += tv[u];
      }
#pragma unroll
      for (int m = 16; m > 0; m >>= 1) v = v + __shfl_xor(v, m, 32);
      if (gln == 0) sk[k] = v;
    }
    __syncthreads();
  }
  if (t != 0) return;
  DevState* st = p.st;
  const float inv = 1.0f / (float)pp.n_mb;  // ppo.rs:374-381
  st->stats[0] = st->ep_kl * inv;
  st->stats[1] = st->ep_surr * inv;
  st->stats[2] = st->ep_vloss * inv;
  st->stats[3] = st->ep_ent * inv;
  st->epochs_run += 1;
  if (kl_on) {
    float kl = 0.f;
    if (p.kl_form == 1) {
      const float R = (float)pp.mb;
      for (int k = 0; k < pp.A; ++k) {
        const float ls_new = p.log_std[k];
        const float d = ls_new - p.log_std_old[k];
        const float ck = 0.5f * (expm1f(-2.0f * d) + 2.0f * d);
        kl += ck + 0.5f * (sk[k] / R) * expf(-2.0f * ls_new);
      }
    } else {
      for (int b = 0; b < p.nkl; ++b) kl += p.kl_part[b];
      kl /= (float)pp.mb;
    }
    st->last_kl = kl;
    if (pp.adaptive_lr) {  // biped_train_gpu.rs:1497-1501
      if (kl > pp.desired_kl * 2.0f)
        st->lr = fmaxf(st->lr / 1.5f, pp.lr_min);
      else if (kl > 0.0f && kl < pp.desired_kl / 2.0f)
        st->lr = fminf(st->lr * 1.5f, pp.lr_max);
    }
    if (pp.early_stop && kl > pp.desired_kl * 5.0f) *p.active = 0;  // :1513-1515
  }
  st->stats[4] = st->lr;
  if (p.begin_next && *p.active) open_epoch(st, pp);
}

// --------------------------------------------------------- GAE / advantages

// zealot-rl/src/ppo.rs:681-703: one thread per env, serial backward scan.
// For T <= kGaeMaxT an env's whole trajectory (rewards, values, dones) is
// loaded into registers before the scan, so the loads are all in flight at
// once instead of one dependent round trip per step; the recurrence is the
// reference's, term for term.
__device__ void gae_body(const GaeArgs& p) {
  if (p.guard && *p.guard == 0) return;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  // T = 0 writes nothing (and the clamped loads below need a step to read).
  if (e >= p.N || p.T <= 0) return;
  float acc = 0.f;
  float next_v = p.last_v[e];
  if (p.T <= kGaeMaxT) {
    // Every load unconditional (steps past T re-read step T - 1), so they
    // issue back to back with one wait.
    float rr[kGaeMaxT], vv[kGaeMaxT];
    uint8_t dd[kGaeMaxT];
#pragma unroll
    for (int i = 0; i < kGaeMaxT; ++i) {
      const long long ii = (long long)min(i, p.T - 1) * p.in_ts + (long long)e * p.in_es;
      rr[i] = p.r[ii];
      vv[i] = p.v[ii];
      dd[i] = p.done[ii];
    }
    float nn[kGaeMaxT];
#pragma unroll
    for (int i = 0; i < kGaeMaxT; ++i) nn[i] = dd[i] ? 0.0f : 1.0f;
#pragma unroll
    for (int i = kGaeMaxT - 1; i >= 0; --i) {
      if (i < p.T) {
        const long long oi = (long long)i * p.out_ts + (long long)e * p.out_es;
        const float delta = rr[i] + p.gamma * next_v * nn[i] - vv[i];
        acc = delta + p.gamma * p.lam * nn[i] * acc;
        p.adv[oi] = acc;
        p.ret[oi] = acc + vv[i];
        next_v = vv[i];
      }
    }
    return;
  }
  for (int i = p.T - 1; i >= 0; --i) {
    const long long ii = (long long)i * p.in_ts + (long long)e * p.in_es;
    const long long oi = (long long)i * p.out_ts + (long long)e * p.out_es;
    const float nt = p.done[ii] ? 0.0f : 1.0f;
    const float vi = p.v[ii];
    const float delta = p.r[ii] + p.gamma * next_v * nt - vi;
    acc = delta + p.gamma * p.lam * nt * acc;
    p.adv[oi] = acc;
    p.ret[oi] = acc + vi;
    next_v = vi;
  }
}

// Advantage normalisation (ppo.rs:343-348 / biped_train_gpu.rs:1010-1016):
// population variance, sd floored at 1e-6. Three launches; every block
// re-derives mean / var from the same partials in the same order.
__device__ void adv_norm_body(const AdvNormArgs& p) {
  __shared__ float red[kThreads];
  __shared__ float bc[2];
  if (p.guard && *p.guard == 0) return;
  const long long lo = (long long)blockIdx.x * p.chunk;
  const long long hi = min(p.n, lo + p.chunk);
  if (p.phase > 0) {
    if (threadIdx.x == 0) {
      float s = 0.f;
      for (int b = 0; b < p.nparts; ++b) s += p.part[b];
      const float mean = s / (float)p.n;
      bc[0] = mean;
      if (p.phase == 2) {
        float q = 0.f;
        for (int b = 0; b < p.nparts; ++b) q += p.part2[b];
        const float var = q / (float)p.n;
        bc[1] = fmaxf(sqrtf(var), 1e-6f);
      }
    }
    __syncthreads();
  }
  if (p.phase == 0) {
    float s = 0.f;
    for (long long i = lo + threadIdx.x; i < hi; i += kThreads) s += p.x[i];
    const float tot = block_sum(s, red);
    if (threadIdx.x == 0) p.part[blockIdx.x] = tot;
  } else if (p.phase == 1) {
    const float mean = bc[0];
    float s = 0.f;
    for (long long i = lo + threadIdx.x; i < hi; i += kThreads) {
      const float d = p.x[i] - mean;
      s += d * d;
    }
    const float tot = block_sum(s, red);
    if (threadIdx.x == 0) p.part2[blockIdx.x] = tot;
  } else {
    const float mean = bc[0], sd = bc[1];
    float* const wb = p.wb ? *p.wb : nullptr;
    for (long long i = lo + threadIdx.x; i < hi; i += kThreads) {
      const float y = (p.x[i] - mean) / sd;
      p.x[i] = y;
      if (wb) wb[i] = y;
    }
  }
}

// ------------------------------------------------------ elementwise utilities

// cuTile elu_backward_ct (src/biped/cutile_gemm.rs:272-286): g *= elu'(y).
__device__ void elu_backward_body(const EluBwdArgs& p) {
  if (p.guard && *p.guard == 0) return;
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= p.rows * p.cols) return;
  const long long r = i / p.cols;
  const int c = (int)(i % p.cols);
  float* gp = p.g + r * p.ldg + c;
  *gp = *gp * elu_grad_from_act(p.y[r * p.ldy + c]);
}

// cuTile row_sum_ct (src/biped/cutile_gemm.rs:290-311): one block per row.
__device__ void row_sum_body(const RowSumArgs& p) {
  __shared__ float red[kThreads];
  if (p.guard && *p.guard == 0) return;
  const int r = blockIdx.x;
  float s = 0.f;
  for (int c = threadIdx.x; c < p.cols; c += kThreads) s += p.x[(long long)r * p.ldx + c];
  const float tot = block_sum(s, red);
  if (threadIdx.x == 0) p.out[r] = tot;
}

// Row gather / pad: dst[r, c] = src[srow, c] for c < cols, 0 for cols <= c < ldd
// when zero_pad (otherwise those columns are left untouched).
__device__ void copy_rows_body(const CopyRowsArgs& p) {
  if (p.guard && *p.guard == 0) return;
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= p.rows * p.ldd) return;
  const long long r = i / p.ldd;
  const int c = (int)(i % p.ldd);
  if (c >= p.cols && !p.zero_pad) return;
  float v = 0.f;
  if (c < p.cols) {
    const long long sr = p.perm ? p.perm[p.row0 + r] : p.row0 + r;
    v = p.src[sr * p.lds + c];
  }
  p.dst[r * p.ldd + c] = v;
}

// Out-of-place transpose (TransposeArgs): reads along a source row and
// writes along a destination row, both coalesced, through a padded LDS tile.
__device__ void transpose_body(const TransposeArgs& p) {
  constexpr int T = kTransposeTile, P = kThreads / T;  // P rows per pass
  __shared__ float tile[T][T + 1];
  const long long i0 = (long long)blockIdx.y * T, j0 = (long long)blockIdx.x * T;
  const int tx = threadIdx.x % T, ty = threadIdx.x / T;
#pragma unroll
  for (int u = 0; u < T / P; ++u) {
    const long long i = i0 + ty + u * P, j = j0 + tx;
    if (i < p.rows && j < p.cols) tile[ty + u * P][tx] = p.src[i * p.lds + j];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < T / P; ++u) {
    const long long j = j0 + ty + u * P, i = i0 + tx;
    if (i < p.rows && j < p.cols) p.dst[j * p.ldd + i] = tile[tx][ty + u * P];
  }
}

// ActorCritic::sample + logp (zealot-rl/src/ppo.rs:314-323, :297-305) with
// the Gaussian noise supplied by the caller, A <= G: a lane group of G lanes
// per row, lane k on action component k (coalesced row reads and writes);
// the logp terms are added in component order by the row's lane 0, as the
// reference's sequential sum does.
template <int G>
__device__ void sample_lanes_body(const SampleArgs& p) {
  constexpr int RPB = kThreads / G;  // rows per block
  __shared__ float s_ls[G], s_sd[G];
  __shared__ float s_term[kThreads];
  if (p.guard && *p.guard == 0) return;
  const int t = threadIdx.x, k = t % G, rr = t / G;
  if (t < G && t < p.A) {
    s_ls[t] = p.log_std[t];
    s_sd[t] = expf(s_ls[t]);
  }
  __syncthreads();
  const long long r = (long long)blockIdx.x * RPB + rr;
  float term = 0.f;
  if (r < p.rows && k < p.A) {
    const float mu = p.mean[r * p.ldm + k];
    const float a = mu + s_sd[k] * p.eps[r * p.lde + k];
    p.action[r * p.lda + k] = a;
    const float d = (a - mu) / s_sd[k];
    term = -0.5f * d * d - s_ls[k] - kLogSqrt2Pi;
  }
  s_term[t] = term;
  __syncthreads();
  if (k == 0 && r < p.rows) {
    float lp = 0.f;
    for (int j = 0; j < p.A; ++j) lp += s_term[rr * G + j];
    p.logp[r] = lp;
  }
}

// Any A: one thread per row.
__device__ void sample_body(const SampleArgs& p) {
  if (p.guard && *p.guard == 0) return;
  const int r = blockIdx.x * kThreads + threadIdx.x;
  if (r >= p.rows) return;
  const float* mu = p.mean + (long long)r * p.ldm;
  const float* ep = p.eps + (long long)r * p.lde;
  float* act = p.action + (long long)r * p.lda;
  for (int k = 0; k < p.A; ++k) {
    const float sd = expf(p.log_std[k]);
    act[k] = mu[k] + sd * ep[k];
  }
  float lp = 0.f;
  for (int k = 0; k < p.A; ++k) {
    const float ls = p.log_std[k];
    const float sd = expf(ls);
    const float d = (act[k] - mu[k]) / sd;
    lp += -0.5f * d * d - ls - kLogSqrt2Pi;
  }
  p.logp[r] = lp;
}

// Batch staging (see StageArgs): every field of a rollout batch copied into
// library-owned batch-major buffers with 16-byte aligned, zero-padded rows;
// feature-major sources ([dim x n], the reference trainer's staging layout,
// src/bin/biped_train_gpu.rs:1029-1068) are transposed through LDS.
__device__ void stage_body(const StageArgs& p) {
  __shared__ float tile[kStageRows][kStageCols + 1];
  if (p.guard && *p.guard == 0) return;
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < p.njobs && b >= p.job[j + 1].blk0) ++j;
  const StageJob& jb = p.job[j];
  const int lb = b - jb.blk0;
  if (lb >= jb.blocks) return;
  const int t = threadIdx.x;
  if (jb.vec) {
    const float* src = p.ptrs->vec[jb.slot];
    const long long base = (long long)lb * kStageVec;
#pragma unroll
    for (int u = 0; u < kStageVec / kThreads; ++u) {
      const long long r = base + u * kThreads + t;
      if (r < p.rows) {
        const long long sr = p.perm ? (long long)p.perm[p.row0 + r] : p.row0 + r;
        jb.dst[r] = src[sr];
      }
    }
    return;
  }
  const float* src = p.ptrs->mat[jb.slot];
  const long long r0 = (long long)(lb / jb.tiles_c) * kStageRows;
  const int c0 = (lb % jb.tiles_c) * kStageCols;
  if (jb.fm) {
    // Read along samples (coalesced in a feature row), write along features.
    const int rr = t % kStageRows, cq = t / kStageRows;
    const long long r = r0 + rr;
    long long sr = 0;
    if (r < p.rows) sr = p.perm ? (long long)p.perm[p.row0 + r] : p.row0 + r;
#pragma unroll
    for (int u = 0; u < kStageCols / (kThreads / kStageRows); ++u) {
      const int c = cq + u * (kThreads / kStageRows);
      const int cg = c0 + c;
      tile[rr][c] = (r < p.rows && cg < jb.cols) ? src[(long long)cg * jb.ld + sr] : 0.f;
    }
    __syncthreads();
    const int c = t % kStageCols, rq = t / kStageCols;
    const int cg = c0 + c;
#pragma unroll
    for (int u = 0; u < kStageRows / (kThreads / kStageCols); ++u) {
      const int rr2 = rq + u * (kThreads / kStageCols);
      const long long r2 = r0 + rr2;
      if (r2 < p.rows && cg < jb.ldd) jb.dst[r2 * jb.ldd + cg] = tile[rr2][c];
    }
  } else {
    const int c = t % kStageCols, rq = t / kStageCols;
    const int cg = c0 + c;
#pragma unroll
    for (int u = 0; u < kStageRows / (kThreads / kStageCols); ++u) {
      const long long r = r0 + rq + u * (kThreads / kStageCols);
      if (r >= p.rows || cg >= jb.ldd) continue;
      float v = 0.f;
      if (cg < jb.cols) {
        const long long sr = p.perm ? (long long)p.perm[p.row0 + r] : p.row0 + r;
        v = src[sr * jb.ld + cg];
      }
      jb.dst[r * jb.ldd + cg] = v;
    }
  }
}

// Per-block sums of squares over a list of tensors (Reduce::SqNorm of every
// gradient tensor, src/bin/biped_train_gpu.rs:1377-1397): block b covers
// chunk b - blk0[j] of tensor j; partial b = its sum (fixed in-block tree).
__device__ void sumsq_multi_body(const SumsqMultiArgs& p) {
  __shared__ float red[kThreads];
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < p.count && b >= p.blk0[j + 1]) ++j;
  const long long lo = (long long)(b - p.blk0[j]) * p.chunk;
  const long long hi = min(p.n[j], lo + p.chunk);
  const float* x = p.x[j];
  float s = 0.f;
  if (((uintptr_t)x & 15u) == 0) {
    const long long hi4 = lo + ((hi - lo) & ~3LL);
    for (long long i = lo + 4 * threadIdx.x; i < hi4; i += 4 * kThreads) {
      const float4 v = *reinterpret_cast<const float4*>(x + i);
      s += v.x * v.x;
      s += v.y * v.y;
      s += v.z * v.z;
      s += v.w * v.w;
    }
    for (long long i = hi4 + threadIdx.x; i < hi; i += kThreads) s += x[i] * x[i];
  } else {
    for (long long i = lo + threadIdx.x; i < hi; i += kThreads) s += x[i] * x[i];
  }
  const float tot = block_sum(s, red);
  if (threadIdx.x == 0) p.part[b] = tot;
}

// One wavefront: the norm from the partials in block order, and the clip
// scale of the trainer's global clip (src/bin/biped_train_gpu.rs:1398-1404):
// max_norm / norm when norm > max_norm, else 1.
__device__ __forceinline__ float clip_scale_of(float sq, float max_norm, float* norm_out) {
  const float norm = sqrtf(sq);
  *norm_out = norm;
  return (max_norm > 0.0f && norm > max_norm) ? max_norm / norm : 1.0f;
}
__device__ void clip_scale_body(const ClipScaleArgs& p) {
  if (threadIdx.x >= 64) return;
  const float sq = wave_sum_strided(p.part, p.nparts, 1);
  if (threadIdx.x != 0) return;
  float norm;
  *p.scale = clip_scale_of(sq, p.max_norm, &norm);
  if (p.norm) *p.norm = norm;
}

// Adam element update of zealot-rl/src/net.rs:240-245 over a list of tensors
// (vortx Adam::step per tensor, src/bin/biped_train_gpu.rs:501-538,
// 1453-1461), the clip scale read from the device.
__device__ void adam_multi_body(const AdamMultiArgs& p) {
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < p.count && b >= p.blk0[j + 1]) ++j;
  const AdamTensor& T = p.t[j];
  const long long i0 = ((long long)(b - p.blk0[j]) * kThreads + threadIdx.x) * 4;
  const bool live = i0 < T.n;
  const bool quad = i0 + 4 <= T.n &&
                    ((((uintptr_t)T.p | (uintptr_t)T.g | (uintptr_t)T.m | (uintptr_t)T.v) & 15u) == 0);
  // The element loads first: they do not depend on the clip scale, so they
  // are in flight while the block takes it.
  float x[4], g[4], m[4], v[4];
  if (quad) {
    const float4 x4 = *reinterpret_cast<const float4*>(T.p + i0);
    const float4 g4 = *reinterpret_cast<const float4*>(T.g + i0);
    const float4 m4 = *reinterpret_cast<const float4*>(T.m + i0);
    const float4 v4 = *reinterpret_cast<const float4*>(T.v + i0);
    x[0] = x4.x, x[1] = x4.y, x[2] = x4.z, x[3] = x4.w;
    g[0] = g4.x, g[1] = g4.y, g[2] = g4.z, g[3] = g4.w;
    m[0] = m4.x, m[1] = m4.y, m[2] = m4.z, m[3] = m4.w;
    v[0] = v4.x, v[1] = v4.y, v[2] = v4.z, v[3] = v4.w;
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool in = i0 + u < T.n;
      x[u] = in ? T.p[i0 + u] : 0.f;
      g[u] = in ? T.g[i0 + u] : 0.f;
      m[u] = in ? T.m[i0 + u] : 0.f;
      v[u] = in ? T.v[i0 + u] : 0.f;
    }
  }
  float sc = 1.0f;
  if (p.part) {
    // Every block: wavefront 0 adds the partials as zk_clip_scale does and
    // lane 0 takes the scale (every thread reaches the barrier).
    __shared__ float s_sc;
    if (threadIdx.x < 64) {
      const float sq = wave_sum_strided(p.part, p.nparts, 1);
      if (threadIdx.x == 0) {
        float norm;
        s_sc = clip_scale_of(sq, p.max_norm, &norm);
        if (b == 0) {
          if (p.scale_out) *p.scale_out = s_sc;
          if (p.norm_out) *p.norm_out = norm;
        }
      }
    }
    __syncthreads();
    sc = s_sc;
  } else if (p.scale) {
    sc = *p.scale;
  }
  if (!live) return;
  const float b1 = p.beta1, b2 = p.beta2, eps = p.eps, lr = p.lr, bc1 = p.bc1, bc2 = p.bc2;
  const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float gr = g[u] * sc;
    m[u] = b1 * m[u] + omb1 * gr;
    v[u] = b2 * v[u] + omb2 * gr * gr;
    x[u] = x[u] - lr * (m[u] / bc1) / (sqrtf(v[u] / bc2) + eps);
  }
  if (quad) {
    *reinterpret_cast<float4*>(T.m + i0) = make_float4(m[0], m[1], m[2], m[3]);
    *reinterpret_cast<float4*>(T.v + i0) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(T.p + i0) = make_float4(x[0], x[1], x[2], x[3]);
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i0 + u < T.n) {
        T.m[i0 + u] = m[u];
        T.v[i0 + u] = v[u];
        T.p[i0 + u] = x[u];
      }
    }
  }
}

__device__ void clamp_body(const ClampArgs& p) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < p.n) p.x[i] = clampf(p.x[i], p.lo, p.hi);
}

}  // namespace zk

#define ZK_KERNEL(NAME, ARGS, BODY) \
  extern "C" __global__ __launch_bounds__(256) void NAME(zk::ARGS p) { zk::BODY(p); }

// One lane group of 32 (A <= 32) or 64 (A <= 64) lanes per sample; separate
// kernels so that the narrow case is not sized for the wide one's registers.
extern "C" __global__ __launch_bounds__(zk::kLossThreads) void zk_actor_loss(zk::ActorLossArgs p) {
  zk::actor_loss_body<32>(p);
}
extern "C" __global__ __launch_bounds__(zk::kLossThreads) void zk_actor_loss_g64(zk::ActorLossArgs p) {
  zk::actor_loss_body<64>(p);
}
ZK_KERNEL(zk_value_loss, ValueLossArgs, value_loss_body)
ZK_KERNEL(zk_sumsq, SumsqArgs, sumsq_body)
ZK_KERNEL(zk_adam, AdamArgs, adam_body)

// All weight and bias gradients of a minibatch step (reduce_all_body) and,
// when tail_block >= 0, the scalar tail of the step in that extra last block.
extern "C" __global__ __launch_bounds__(zk::kReduceAllThreads) void zk_reduce_all(zk::ReduceAllArgs a) {
  if (a.guard && *a.guard == 0) return;
  if ((int)blockIdx.x == a.tail_block)
    zk::minibatch_tail_body(a.tail);
  else
    zk::reduce_all_body(a);
}
ZK_KERNEL(zk_epoch_begin, EpochBeginArgs, epoch_begin_body)
ZK_KERNEL(zk_kl, KlArgs, kl_body)
extern "C" __global__ __launch_bounds__(zk::kFinalizeThreads) void zk_epoch_end(zk::EpochEndArgs p) {
  zk::epoch_end_body(p);
}
ZK_KERNEL(zk_gae, GaeArgs, gae_body)
ZK_KERNEL(zk_adv_norm, AdvNormArgs, adv_norm_body)
ZK_KERNEL(zk_elu_backward, EluBwdArgs, elu_backward_body)
ZK_KERNEL(zk_row_sum, RowSumArgs, row_sum_body)
ZK_KERNEL(zk_copy_rows, CopyRowsArgs, copy_rows_body)
ZK_KERNEL(zk_transpose, TransposeArgs, transpose_body)
ZK_KERNEL(zk_sample, SampleArgs, sample_body)
extern "C" __global__ __launch_bounds__(256) void zk_sample_g32(zk::SampleArgs p) { zk::sample_lanes_body<32>(p); }
extern "C" __global__ __launch_bounds__(256) void zk_sample_g64(zk::SampleArgs p) { zk::sample_lanes_body<64>(p); }
ZK_KERNEL(zk_clamp, ClampArgs, clamp_body)
ZK_KERNEL(zk_stage, StageArgs, stage_body)
ZK_KERNEL(zk_sumsq_multi, SumsqMultiArgs, sumsq_multi_body)
ZK_KERNEL(zk_clip_scale, ClipScaleArgs, clip_scale_body)
ZK_KERNEL(zk_adam_multi, AdamMultiArgs, adam_multi_body)
