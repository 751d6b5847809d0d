// head.hip — the output layer of the actor and the critic fused with the PPO
// losses of one minibatch (zealot-rl/src/ppo.rs:410-451, net.rs:88-140 for
// the last layer): per tile of kHeadRows rows, the head forward, the actor's
// clipped surrogate / the critic's clipped value loss, the head's data
// gradient times ELU' of the last hidden activations (dL/dz of the last
// hidden layer), and the head's weight and bias gradients as per-block
// partials. The activations of a tile are read once into LDS (zk_head_fwd*:
// computed there from the layer below, so that layer's output never goes to
// HBM) and every intermediate (means, their gradients) stays there. All sums
// run in a fixed order, so the results are the same on every run.
#pragma once
#include "common.hip"
#include "ppo_kernels.hip"

namespace zk {

// Block barrier for LDS only: this wave's LDS writes complete, then
// s_barrier. Unlike __syncthreads it does not wait for outstanding global
// loads and stores, so the loss inputs stay in flight across the forward and
// the stores drain in the background.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

constexpr int kHeadGroups = kHeadThreads / 32;  // 32-lane loss groups
constexpr int kHeadPitch = kHeadMaxHidden + 4;  // LDS row pitch of the activation tile
constexpr int kHeadDPitch = kHeadMaxActions + 4;
constexpr int kHeadRed = kHeadGroups * 34 > kHeadThreads ? kHeadGroups * 34 : kHeadThreads;
constexpr int kHeadLds =
    kHeadRows * kHeadPitch + kHeadMaxActions * kHeadPitch + kHeadRows * kHeadDPitch + kHeadRed;
static_assert(kHeadRows == 64 && kHeadMaxHidden == 128 && kHeadMaxActions == 32,
              "wave-to-tile mapping of zk_head");

// A float4 with the components at column c + i >= lim (or all, if !row_ok)
// replaced by 0.
__device__ __forceinline__ float4 quad_or_zero(float4 v, bool row_ok, int c, int lim) {
  v.x = row_ok && c < lim ? v.x : 0.f;
  v.y = row_ok && c + 1 < lim ? v.y : 0.f;
  v.z = row_ok && c + 2 < lim ? v.z : 0.f;
  v.w = row_ok && c + 3 < lim ? v.w : 0.f;
  return v;
}

// Rows [r0, r0 + nr) of x into sx (kHeadRows x kHeadPitch), zero past nr
// rows and past H columns (up to kHeadMaxHidden); nr >= 1. Every thread's
// loads are unconditional, from clamped in-range addresses (a float4 at a
// column < H stays inside the row's 4-aligned stride), so they all issue
// before the first wait; out-of-range values are replaced by 0 afterwards.
constexpr int kHeadQPR = kHeadMaxHidden / 4;                      // float4 quads per row
constexpr int kHeadTileQuads = kHeadRows * kHeadQPR / kHeadThreads;  // per thread
static_assert(kHeadRows * kHeadQPR % kHeadThreads == 0, "whole quads per thread");
__device__ __forceinline__ void head_tile_issue(const HeadNet& q, long long r0, int nr,
                                                float4 (&v)[kHeadTileQuads]) {
  const int c_last = (q.H - 1) & ~3;
  const float* base = q.x + r0 * q.ldx;  // uniform; 32-bit offsets within the tile
#pragma unroll
  for (int u = 0; u < kHeadTileQuads; ++u) {
    const int i = threadIdx.x + kHeadThreads * u, r = i / kHeadQPR, c = (i % kHeadQPR) * 4;
    v[u] = *reinterpret_cast<const float4*>(base + (min(r, nr - 1) * q.ldx + min(c, c_last)));
  }
}
__device__ __forceinline__ void head_tile_store(const HeadNet& q, int nr, const float4 (&v)[kHeadTileQuads],
                                                float* sx) {
#pragma unroll
  for (int u = 0; u < kHeadTileQuads; ++u) {
    const int i = threadIdx.x + kHeadThreads * u, r = i / kHeadQPR, c = (i % kHeadQPR) * 4;
    *reinterpret_cast<float4*>(sx + r * kHeadPitch + c) = quad_or_zero(v[u], r < nr, c, q.H);
  }
}
__device__ __forceinline__ void head_load_tile(const HeadNet& q, long long r0, int nr, float* sx) {
  float4 v[kHeadTileQuads];
  head_tile_issue(q, r0, nr, v);
  head_tile_store(q, nr, v, sx);
}

// zk_head_fwd*: rows [r0, r0 + kHeadRows) of the last hidden layer's output,
// ELU(x2 . w2^T + b2), computed into sx by a 64 x 128 GEMM tile whose 32-wide
// k-tiles are staged in smem (sx overlaps that staging: the tile is written
// after the k-loop's last barrier). All 64 rows and 128 columns are written;
// rows past the minibatch and columns past H come from zero operands, so they
// are finite, and the phases that follow give them zero weight. EXACT: rows,
// H = 128 and k2 are whole tiles (the host checks), no clamps or masks.
constexpr int kHeadFwdBK = 32;
static_assert(gemm_smem_floats<true, true, kHeadRows, kHeadMaxHidden, kHeadFwdBK, 2, 4, true>() <= kHeadLds,
              "the forward tile's staging fits the head's LDS");
template <bool EXACT>
__device__ __forceinline__ void head_forward_tile(const HeadNet& q, long long rows, long long r0,
                                                  float* smem, float* sx) {
  GemmArgs a{};
  a.A = q.x2;
  a.lda = q.ldx2;
  a.B = q.w2;
  a.ldb = q.ldw2;
  a.bias = q.b2;
  a.M = (int)rows;
  a.N = q.H;
  a.K = q.k2;
  a.ldc = kHeadPitch;
  a.epi = kEpiBiasN;
  a.act = 1;
  a.vecA = a.vecB = 1;
  a.kt_per_split = (q.k2 + kHeadFwdBK - 1) / kHeadFwdBK;
  a.nsplit = 1;
  gemm_body<true, true, kHeadRows, kHeadMaxHidden, kHeadFwdBK, 2, 4, true, false, EXACT, true>(
      smem, a, 0, (int)(r0 / kHeadRows), 0, sx);
}

// Sum over a row's 32 components in component order, every lane of the
// 32-lane group getting the result: lane k stores its term in the row's LDS
// slot k (components >= A hold 0, and adding 0 changes no sum), the group's
// first lane reads the row back as 8 float4 loads and adds them in order, and
// the two groups' sums (lanes 0 and 32 of the wavefront) are broadcast with
// v_readlane. LDS instructions of one wavefront execute in order, so no
// barrier is needed; one reading lane per group instead of 32 keeps the LDS
// traffic of the losses at 1/32.
__device__ __forceinline__ float row_sum_ordered(float* srow, int k, float term) {
  srow[k] = term;
  float s = 0.f;
  if (k == 0) {
#pragma unroll
    for (int c = 0; c < kHeadMaxActions / 4; ++c) {
      const float4 v = *reinterpret_cast<const float4*>(srow + 4 * c);
      s += v.x;
      s += v.y;
      s += v.z;
      s += v.w;
    }
  }
  const float s0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), 0));
  const float s1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), 32));
  return (threadIdx.x & 32) ? s1 : s0;
}

// FWD: 0 reads the tile of the last hidden activations; 1 (masked) / 2
// (exact-fit) computes it (head_forward_tile).
template <int FWD>
__device__ void head_actor(const HeadArgs& p, float* smem) {
  const HeadNet& q = p.net[0];
  float* sx = smem;                                      // activations [R x pitch]
  float* sw = sx + kHeadRows * kHeadPitch;               // weights [32 x pitch], rows >= A zero
  float* sd = sw + kHeadMaxActions * kHeadPitch;         // means, then dL/dmean [R x dpitch]
  float* sred = sd + kHeadRows * kHeadDPitch;            // [groups][34]
  int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  int lr = lane & 15, lg = lane >> 4;
  const int A = p.A, H = q.H;

  // The head weights, rows >= A and columns >= H zero (loads as in
  // head_load_tile). With FWD the forward tile's staging overwrites sw, so
  // they are read after the tile's forward.
  constexpr int WQPR = kHeadMaxHidden / 4;
  constexpr int WNQ = kHeadMaxActions * WQPR / kHeadThreads;
  static_assert(kHeadMaxActions * WQPR % kHeadThreads == 0, "whole quads per thread");
  float4 wv[WNQ];
  auto load_weights = [&]() {
    const int c_last = (H - 1) & ~3;
#pragma unroll
    for (int u = 0; u < WNQ; ++u) {
      const int i = t + kHeadThreads * u, m = i / WQPR, c = (i % WQPR) * 4;
      wv[u] = *reinterpret_cast<const float4*>(q.w + (long long)min(m, A - 1) * q.ldw + min(c, c_last));
    }
  };
  if constexpr (FWD == 0) load_weights();
  auto store_weights = [&]() {
#pragma unroll
    for (int u = 0; u < WNQ; ++u) {
      const int i = t + kHeadThreads * u, m = i / WQPR, c = (i % WQPR) * 4;
      *reinterpret_cast<float4*>(sw + m * kHeadPitch + c) = quad_or_zero(wv[u], m < A, c, H);
    }
  };
  if constexpr (FWD == 0) store_weights();

  // Loss lanes: 16 groups of 32, lane k on action component k.
  int grp = t >> 5, k = t & 31;
  bool on = k < A;
  // Per-lane loss constants (with FWD set after each tile's forward, so that
  // they hold no registers during its GEMM).
  float ls = 0.f, sdv = 0.f, inv_var = 0.f, inv_sd = 0.f;
  auto loss_consts = [&]() {
    ls = on ? p.log_std[k] : 0.f;
    sdv = expf(ls);
    inv_var = expf(-2.0f * ls);
    inv_sd = expf(-ls);
  };
  if constexpr (FWD == 0) loss_consts();
  const float lo = 1.0f - p.clip, hi = 1.0f + p.clip;
  float gacc = 0.f, sacc = 0.f, kacc = 0.f;
  float klacc = 0.f;  // sum of (mean - mean_old)^2 of component k over the group's rows
  float dbias = 0.f;  // thread t < 32: bias gradient of component t
  floatx4 wacc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
  // Wave-to-tile mapping: 16-row tile rt = wave % 4; forward components
  // 16 * (wave / 4) ..; data-gradient columns 64 * (wave / 4) ..; weight
  // gradient columns 16 * wave ...
  int rt = wave & 3, half = wave >> 2;
  int mf = 16 * half + lr;  // this lane's forward component
  float bias_f = 0.f;
  auto load_bias = [&]() { bias_f = mf < A ? q.b[min(mf, A - 1)] : 0.f; };
  if constexpr (FWD == 0) load_bias();

  struct In {
    float act, lpo, adv, mo;
  };
  constexpr int RG = kHeadRows / kHeadGroups;  // rows per loss group
  const long long ntiles = (p.rows + kHeadRows - 1) / kHeadRows;
  // With FWD a block takes one tile (the host lays the grid out so), which
  // leaves the loop's accumulators at zero while the tile's GEMM runs.
  const int tpb = FWD ? 1 : p.tiles_per_block;
  for (int tt = 0; tt < tpb; ++tt) {
    const long long tile = blockIdx.x + (long long)tt * gridDim.x;
    if (tile >= ntiles) break;  // uniform
    long long r0 = tile * kHeadRows;
    int nr = (int)min((long long)kHeadRows, p.rows - r0);
    // Loss inputs of the group's rows, in flight during the tile load and
    // the forward (group g takes rows g, g + 16, ...; with FWD, issued after
    // the tile's GEMM so that they hold no registers during it).
    // Rows past nr read the last row's inputs (the loss skips those rows),
    // so every load is unconditional in the row and the sample indices of
    // a shuffled minibatch are all in flight before the first wait.
    In in[RG];
    auto load_inputs = [&]() {
      long long sidx[RG];
#pragma unroll
      for (int j = 0; j < RG; ++j) {
        const long long rr = p.row0 + r0 + min(grp + kHeadGroups * j, nr - 1);
        sidx[j] = p.perm ? (long long)p.perm[rr] : rr;
      }
#pragma unroll
      for (int j = 0; j < RG; ++j) {
        const long long s = sidx[j];
        In x;
        x.act = on ? p.action[s * p.ldact + k] : 0.f;
        x.lpo = p.logp_old[s];
        x.adv = p.adv[s];
        x.mo = (p.mean_old && on) ? p.mean_old[s * p.ldmo + k] : 0.f;
        in[j] = x;
      }
    };
    if constexpr (FWD == 0) load_inputs();
    lds_barrier();  // the previous tile's LDS reads are done
    if constexpr (FWD == 0) {
      head_load_tile(q, r0, nr, sx);
    } else {
      head_forward_tile<FWD == 2>(q, p.rows, r0, smem, sx);
      {
        // The tile's row and the thread's indices made opaque here, so that
        // the compiler computes the addresses of the phases below after the
        // GEMM instead of holding them in registers across it (which spills).
        int ti = (int)tile;
        asm volatile("" : "+s"(ti));
        r0 = (long long)ti * kHeadRows;
        nr = (int)min((long long)kHeadRows, p.rows - r0);
        int tv = threadIdx.x;
        asm volatile("" : "+v"(tv));
        t = tv;
        lane = t & 63;
        wave = t >> 6;
        lr = lane & 15;
        lg = lane >> 4;
        grp = t >> 5;
        k = t & 31;
        on = k < A;
        rt = wave & 3;
        half = wave >> 2;
        mf = 16 * half + lr;
      }
      load_weights();
      store_weights();
      load_inputs();
      loss_consts();
      load_bias();
    }
    lds_barrier();

    // Head forward: rows of tile rt, components 16 * half ...; the k range
    // in two interleaved chains (even and odd 16-wide chunks) added at the end.
    {
      floatx4 acc2[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int c16 = 0; c16 < kHeadMaxHidden / 16; ++c16) {
        const float4 af = *reinterpret_cast<const float4*>(sx + (16 * rt + lr) * kHeadPitch + 16 * c16 + 4 * lg);
        const float4 bf = *reinterpret_cast<const float4*>(sw + (16 * half + lr) * kHeadPitch + 16 * c16 + 4 * lg);
        floatx4& acc = acc2[c16 & 1];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, bf.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, bf.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, bf.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, bf.w, acc, 0, 0, 0);
      }
      const int m = mf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * rt + 4 * lg + r;
        const float mu = m < A ? (acc2[0][r] + acc2[1][r]) + bias_f : 0.f;
        sd[row * kHeadDPitch + m] = mu;
        if (m < A && row < nr) q.out[(r0 + row) * q.ldo + m] = mu;
      }
    }
    lds_barrier();

    // Losses (ppo.rs:411-432, as zk_actor_loss).
    {
#pragma unroll
      for (int j = 0; j < RG; ++j) {
        const int row = grp + kHeadGroups * j;
        if (row >= nr) {  // group-uniform
          sd[row * kHeadDPitch + k] = 0.f;
          continue;
        }
        float* srow = sd + row * kHeadDPitch;
        const float mu = srow[k];
        const float act = in[j].act;
        const float dz = (act - mu) / sdv;
        const float lp = row_sum_ordered(srow, k, on ? -0.5f * dz * dz - ls - kLogSqrt2Pi : 0.f);
        const float ratio = expf(lp - in[j].lpo);
        const float a = in[j].adv;
        const float surr = fminf(ratio * a, clampf(ratio, lo, hi) * a);
        const bool clipped = (a >= 0.0f && ratio > hi) || (a < 0.0f && ratio < lo);
        float gm = 0.f, cc = 0.f;
        if (!clipped) {
          const float d = act - mu;
          gm = -(a * ratio * d * inv_var) * p.scale;
          const float dls = a * ratio * ((d * d) * inv_var - 1.0f);
          cc = -dls * p.scale;
        }
        cc += -p.entropy_coef * p.scale;
        if (on) gacc += cc;
        sacc += surr * p.scale;
        if (p.mean_old) {
          const float y = (mu - in[j].mo) * inv_sd;
          // The mean-only KL (ActorCritic::kl, ppo.rs:327-334) is a statistic:
          // a fixed butterfly over the group is enough (every lane ends with
          // the same bits: each step adds two equal-valued partners).
          float kt = on ? 0.5f * (y * y) : 0.f;
#pragma unroll
          for (int m = 16; m > 0; m >>= 1) kt = kt + __shfl_xor(kt, m, 32);
          kacc += kt * p.scale;
          if (p.kl_part && on) {
            const float dmu = mu - in[j].mo;
            klacc += dmu * dmu;
          }
        }
        srow[k] = on ? gm : 0.f;  // the group's own row: no other reader yet
      }
    }
    lds_barrier();

    // Data gradient of the head times ELU' of the activations: rows of tile
    // rt, hidden columns 64 * half ...
    {
      constexpr int NJ = kHeadMaxHidden / 32;
      floatx4 dacc[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) dacc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c16 = 0; c16 < kHeadMaxActions / 16; ++c16) {
        const float4 af = *reinterpret_cast<const float4*>(sd + (16 * rt + lr) * kHeadDPitch + 16 * c16 + 4 * lg);
        const float* wr = sw + (16 * c16 + 4 * lg) * kHeadPitch + 64 * half + lr;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          dacc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, wr[16 * j], dacc[j], 0, 0, 0);
          dacc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, wr[kHeadPitch + 16 * j], dacc[j], 0, 0, 0);
          dacc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, wr[2 * kHeadPitch + 16 * j], dacc[j], 0, 0, 0);
          dacc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, wr[3 * kHeadPitch + 16 * j], dacc[j], 0, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int n = 64 * half + 16 * j + lr;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * rt + 4 * lg + r;
          if (row < nr && n < H)
            q.dz[(r0 + row) * q.ldz + n] = dacc[j][r] * elu_grad_from_act(sx[row * kHeadPitch + n]);
        }
      }
    }

    // Weight gradient partial dW += dmean^T . x over this tile's rows: wave w
    // takes hidden columns 16w..16w+15; the bias gradient is the column sum.
#pragma unroll
    for (int r16 = 0; r16 < kHeadRows / 16; ++r16) {
      float av[2][4], bv[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int row = 16 * r16 + 4 * lg + c;
#pragma unroll
        for (int i = 0; i < 2; ++i) av[i][c] = sd[row * kHeadDPitch + 16 * i + lr];
        bv[c] = sx[row * kHeadPitch + 16 * wave + lr];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          wacc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][c], bv[c], wacc[i], 0, 0, 0);
    }
    if (t < kHeadMaxActions)
      for (int row = 0; row < kHeadRows; ++row) dbias += sd[row * kHeadDPitch + t];
  }

  // Partials of this block.
  const int blk = blockIdx.x, nblk = gridDim.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int n = 16 * wave + lr;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * i + 4 * lg + r;
      if (m < A && n < H) q.wpart[((long long)blk * A + m) * H + n] = wacc[i][r];
    }
  }
  if (t < A) q.bpart[(long long)blk * A + t] = dbias;
  sred[grp * 34 + k] = gacc;
  if (k == 0) {
    sred[grp * 34 + 32] = sacc;
    sred[grp * 34 + 33] = kacc;
  }
  lds_barrier();
  if (t < A) {
    float g = 0.f;
    for (int j = 0; j < kHeadGroups; ++j) g += sred[j * 34 + t];
    p.gls_part[(long long)t * nblk + blk] = g;
  } else if (t == 64 || t == 65) {
    const int qq = t - 64;
    float v = 0.f;
    for (int j = 0; j < kHeadGroups; ++j) v += sred[j * 34 + 32 + qq];
    p.astat_part[(long long)qq * nblk + blk] = v;
  }
  if (p.kl_part) {  // per-component sums for the trainer's full-Gaussian KL
    lds_barrier();
    sred[grp * 34 + k] = klacc;
    lds_barrier();
    if (t < A) {
      float v = 0.f;
      for (int j = 0; j < kHeadGroups; ++j) v += sred[j * 34 + t];
      p.kl_part[(long long)t * nblk + blk] = v;
    }
  }
}

template <int FWD>
__device__ void head_critic(const HeadArgs& p, float* smem) {
  const HeadNet& q = p.net[1];
  float* sx = smem;
  float* sw = sx + kHeadRows * kHeadPitch;         // w[0..128), zero past H
  float* sdv = sw + kHeadMaxActions * kHeadPitch;  // dL/dvalue per row
  float* sred = sdv + kHeadRows * kHeadDPitch;     // [4][128] weight-gradient quarters, [8] wave sums
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int H = q.H;
  // Weights, bias and the first tile's loads go out together (the loads are
  // unconditional, from clamped in-range addresses, as in head_tile_issue).
  const float wt = t < kHeadMaxHidden ? q.w[min(t, H - 1)] : 0.f;
  const float bias = q.b[0];
  float vacc = 0.f, dw = 0.f, db = 0.f;
  const long long ntiles = (p.rows + kHeadRows - 1) / kHeadRows;
  constexpr int U = kHeadThreads / kHeadRows;  // lanes per row (8)
  static_assert(kHeadThreads == 4 * kHeadMaxHidden, "four row quarters per weight-gradient column");
  const int row = t / U, u = t % U;
  const int cb = blockIdx.x, cbn = p.critic_blocks;
  if (cb >= cbn) return;  // uniform: a block of the actor's grid with no critic tile
  // Tiles cb, cb + cbn, ...: each tile's loads are issued while the previous
  // tile is worked on (cb < ntiles: cbn = ceil(ntiles / critic_tiles)).
  float4 xv[kHeadTileQuads];
  if constexpr (FWD == 0)
    head_tile_issue(q, (long long)cb * kHeadRows,
                    (int)min((long long)kHeadRows, p.rows - (long long)cb * kHeadRows), xv);
  const int ctl = p.critic_tiles;
  for (int tt = 0; tt < ctl; ++tt) {
    const long long tile = cb + (long long)tt * cbn;
    if (tile >= ntiles) break;  // uniform
    const long long r0 = tile * kHeadRows;
    const int nr = (int)min((long long)kHeadRows, p.rows - r0);
    // Loss inputs, in flight during the value (rows past nr read the last
    // row's; they are not used).
    float vo = 0.f, R = 0.f;
    if (u == 0) {
      const long long rr = p.row0 + r0 + min(row, nr - 1);
      const long long sidx = p.perm ? (long long)p.perm[rr] : rr;
      vo = p.value_old[sidx];
      R = p.ret[sidx];
    }
    if (FWD == 0 && tt == 0 && t < kHeadMaxHidden) sw[t] = t < H ? wt : 0.f;
    lds_barrier();  // the previous tile's LDS reads are done
    if constexpr (FWD == 0) {
      head_tile_store(q, nr, xv, sx);
      const long long next = tile + cbn;
      if (tt + 1 < p.critic_tiles && next < ntiles)
        head_tile_issue(q, next * kHeadRows, (int)min((long long)kHeadRows, p.rows - next * kHeadRows), xv);
    } else {  // the staging of the tile's forward overwrites sw
      head_forward_tile<FWD == 2>(q, p.rows, r0, smem, sx);
      if (t < kHeadMaxHidden) sw[t] = t < H ? wt : 0.f;
    }
    lds_barrier();
    // value = b + sum_k w_k x_k: U lanes per row, lane u on columns u, u + U,
    // ..., then the U partial sums in lane order.
    {
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < kHeadMaxHidden / U; ++i) part += sx[row * kHeadPitch + u + U * i] * sw[u + U * i];
      const int l0 = lane & ~(U - 1);
      float ps[U];
#pragma unroll
      for (int i = 0; i < U; ++i) ps[i] = __shfl(part, l0 + i, 64);
      if (u == 0) {
        float dv = 0.f;
        if (row < nr) {
          float sum = ps[0];
#pragma unroll
          for (int i = 1; i < U; ++i) sum += ps[i];
          const float v = bias + sum;
          q.out[(r0 + row) * q.ldo] = v;
          // ppo.rs:436-450, as zk_value_loss.
          const float vc = vo + clampf(v - vo, -p.clip, p.clip);
          const float lu = (v - R) * (v - R);
          const float lc = (vc - R) * (vc - R);
          float vloss, g;
          if (lc > lu) {
            vloss = lc;
            g = 2.0f * (vc - R);
          } else {
            vloss = lu;
            g = 2.0f * (v - R);
          }
          vacc += vloss * p.scale;
          dv = p.value_coef * g * p.scale;
        }
        sdv[row] = dv;
      }
    }
    lds_barrier();
    // dL/dz = (dv * w) * ELU'(x), four columns per thread (the dz rows are
    // 16-byte aligned: ldz is a multiple of 4).
#pragma unroll
    for (int uq = 0; uq < kHeadTileQuads; ++uq) {
      const int e = t + kHeadThreads * uq;
      const int rr = e / kHeadQPR, n = (e % kHeadQPR) * 4;
      const float d = sdv[rr];
      const float4 xr = *reinterpret_cast<const float4*>(sx + rr * kHeadPitch + n);
      const float4 wr = *reinterpret_cast<const float4*>(sw + n);
      float4 o;
      o.x = (d * wr.x) * elu_grad_from_act(xr.x);
      o.y = (d * wr.y) * elu_grad_from_act(xr.y);
      o.z = (d * wr.z) * elu_grad_from_act(xr.z);
      o.w = (d * wr.w) * elu_grad_from_act(xr.w);
      if (rr < nr && n < H) {
        float* dst = q.dz + (r0 + rr) * q.ldz + n;
        if (n + 4 <= H) {
          *reinterpret_cast<float4*>(dst) = o;
        } else {
          dst[0] = o.x;
          if (n + 1 < H) dst[1] = o.y;
          if (n + 2 < H) dst[2] = o.z;
        }
      }
    }
    // Weight gradient of this tile: column c = t % 128 over the row quarter
    // t / 128 (16 rows, in row order), the quarters then added in order; the
    // bias gradient by the last thread over all rows in row order.
    {
      const int c = t % kHeadMaxHidden, qr = t / kHeadMaxHidden;
      float pq = 0.f;
#pragma unroll
      for (int r = 0; r < kHeadRows / 4; ++r) {
        const int rr = (kHeadRows / 4) * qr + r;
        pq += sdv[rr] * sx[rr * kHeadPitch + c];
      }
      if (t == kHeadThreads - 1)
        for (int rr = 0; rr < kHeadRows; ++rr) db += sdv[rr];
      sred[qr * kHeadMaxHidden + c] = pq;
      lds_barrier();
      if (t < kHeadMaxHidden) {
        const float* qs = sred + t;
        dw += ((qs[0] + qs[kHeadMaxHidden]) + qs[2 * kHeadMaxHidden]) + qs[3 * kHeadMaxHidden];
      }
    }
  }
  const int blk = blockIdx.x;
  if (t < H) q.wpart[(long long)blk * H + t] = dw;
  if (t == kHeadThreads - 1) q.bpart[blk] = db;
  // Value-loss sum: each wave's U-strided row lanes in lane order, then the
  // waves in order.
  float ws = 0.f;
#pragma unroll
  for (int i = 0; i < 64 / U; ++i) ws += __shfl(vacc, U * i, 64);
  lds_barrier();  // the weight-gradient quarters are read
  if (lane == 0) sred[wave] = ws;
  lds_barrier();
  if (t == 0) {
    float tot = 0.f;
    for (int w = 0; w < kHeadThreads / 64; ++w) tot += sred[w];
    p.vstat_part[blk] = tot;
  }
}

}  // namespace zk

// Held to four waves per SIMD (two blocks of eight wavefronts per CU, which
// the LDS footprint allows): at most 128 VGPRs. zk_head reads the last hidden
// activations; zk_head_fwd (masked) and zk_head_fwd_x (exact-fit) compute
// them from the layer below (HeadNet::x2 / w2 / b2).
#define ZK_HEAD(NAME, FWD)                                                          \
  extern "C" __global__ __launch_bounds__(zk::kHeadThreads)                         \
  __attribute__((amdgpu_waves_per_eu(4))) void NAME(zk::HeadArgs p) {              \
    __shared__ __align__(16) float smem[zk::kHeadLds];                              \
    if (p.guard && *p.guard == 0) return;                                           \
    if (blockIdx.z == 0)                                                            \
      zk::head_actor<FWD>(p, smem);                                                 \
    else                                                                            \
      zk::head_critic<FWD>(p, smem);                                                \
  }
ZK_HEAD(zk_head, 0)
ZK_HEAD(zk_head_fwd, 1)
ZK_HEAD(zk_head_fwd_x, 2)
