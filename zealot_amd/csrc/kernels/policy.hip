// policy.hip — one rollout step of the policy (and optionally the value) in
// one launch: GpuPolicy::forward (src/biped/gpu_policy.rs:210-248) with the
// trainer's sampling (src/bin/biped_train_gpu.rs:910-930). At a rollout's
// few thousand rows the per-layer GEMM launches are latency-bound; here a
// block takes kPolicyRows rows through every layer with the activations in
// LDS, reading each layer's weights from L2 in the fragment-major copy that
// zk_policy_pack writes (a wavefront's load of one tile's 16-wide chunk is
// 1 KB of consecutive floats instead of 64 bytes of each of 16 weight rows).
//
// Every value is computed as on the multi-launch path: the normalisation is
// Normalizer::normalize's expression (ppo.rs:198-205), each layer sums its
// reduction index in 16-wide chunks with lane group s of MFMA step c on
// index k0 + 4 s + c (the order of the tiled and narrow GEMM kernels), adds
// the bias after the sum and applies ELU to the hidden layers, and the
// log-probability adds its terms in component order.
#pragma once
#include "common.hip"

namespace zk {

constexpr int kPolicyPitch = kPolicyMaxWidth + 4;  // LDS row pitch of an activation tile
constexpr int kPolicyWaves = kPolicyThreads / 64;
constexpr int kPolicyMaxTiles = kPolicyMaxWidth / 16 / kPolicyWaves;  // 16-column tiles per wave
constexpr int kPolicyPass = 2;  // 16-wide chunks whose loads are issued together
static_assert(kPolicyRows == 16 && kPolicyThreads >= 32 * kPolicyRows, "one 16-row MFMA tile; a 32-lane group per row");

__device__ void policy_body(const PolicyArgs& p) {
  __shared__ __align__(16) float act[2][kPolicyRows * kPolicyPitch];
  __shared__ float s_mu[kPolicyMaxWidth], s_sd[kPolicyMaxWidth];
  __shared__ float s_term[kPolicyThreads];
  __shared__ float s_ls[32], s_sdv[32];
  const PolicyNet& q = p.net[blockIdx.y];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const long long r0 = (long long)blockIdx.x * kPolicyRows;
  const int nr = (int)min((long long)kPolicyRows, p.rows - r0);
  const int od = q.dims[0];
  const int k0w = (od + 15) & ~15;  // layer 0's reduction width (zero past od)

  // Inputs: rows past nr and columns in [od, k0w) are zero.
  if (q.norm) {
    const float count = q.norm[2 * od];
    for (int c = t; c < od; c += kPolicyThreads) {
      s_mu[c] = q.norm[c];
      s_sd[c] = sqrtf(fmaxf(q.norm[od + c] / count, 1e-8f));
    }
    __syncthreads();
  }
  for (int e = t; e < kPolicyRows * k0w; e += kPolicyThreads) {
    const int row = e / k0w, c = e - row * k0w;
    float v = 0.f;
    if (row < nr && c < od) {
      const float x = q.x[(r0 + row) * q.ldx + c];
      v = q.norm ? clampf((x - s_mu[c]) / s_sd[c], -5.0f, 5.0f) : x;
    }
    act[0][row * kPolicyPitch + c] = v;
  }
  __syncthreads();

  int cur = 0;
  for (int l = 0; l < q.L; ++l) {
    const int K = l == 0 ? k0w : q.dims[l];
    const int N = q.dims[l + 1];
    const bool last = l == q.L - 1;
    const float* Wp = q.wp + q.wp_off[l];
    const float* bias = p.params + q.b_off[l];
    const float* src = act[cur];
    float* dst = act[cur ^ 1];
    const int nt = (N + 15) / 16;
    // This wave's 16-column tiles: slots wave, wave + kPolicyWaves, ... < nt,
    // slot s on tile (s + rot) % nt, rotated per block so that concurrent
    // blocks read different weight tiles (measured within 1 % of no
    // rotation). The weight loads go out one round per kPolicyPass chunks.
    const int rot = (int)(blockIdx.x % (unsigned)nt);
    auto tile_of = [&](int u) {
      const int s = wave + kPolicyWaves * u + rot;
      return s >= nt ? s - nt : s;
    };
    floatx4 acc[kPolicyMaxTiles];
    // 32-bit offsets from the uniform Wp: tile T's chunk c is the 256 floats
    // at (T * kc + c) * 256, this lane's float4 at 4 * lane within them.
    const int kc = K / 16;
    int toff[kPolicyMaxTiles];
#pragma unroll
    for (int u = 0; u < kPolicyMaxTiles; ++u) {
      acc[u] = floatx4{0.f, 0.f, 0.f, 0.f};
      toff[u] = tile_of(u) * kc * 256 + 4 * lane;
    }
    if (wave < nt) {  // uniform over the wavefront
      for (int kp = 0; kp < K; kp += 16 * kPolicyPass) {
        float4 av[kPolicyPass], bv[kPolicyPass][kPolicyMaxTiles];
#pragma unroll
        for (int j = 0; j < kPolicyPass; ++j) {
          const int k = kp + 16 * j + 4 * lg;
          const bool in = kp + 16 * j < K;  // uniform: K % 16 == 0
          av[j] = in ? *reinterpret_cast<const float4*>(src + lr * kPolicyPitch + k) : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int u = 0; u < kPolicyMaxTiles; ++u)
            bv[j][u] = in && wave + kPolicyWaves * u < nt
                           ? *reinterpret_cast<const float4*>(Wp + (toff[u] + 16 * (kp + 16 * j)))
                           : float4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < kPolicyPass; ++j) {
          if (kp + 16 * j >= K) break;
#pragma unroll
          for (int u = 0; u < kPolicyMaxTiles; ++u) {
            if (wave + kPolicyWaves * u >= nt) break;
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].x, bv[j][u].x, acc[u], 0, 0, 0);
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].y, bv[j][u].y, acc[u], 0, 0, 0);
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].z, bv[j][u].z, acc[u], 0, 0, 0);
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].w, bv[j][u].w, acc[u], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kPolicyMaxTiles; ++u) {
        const int n = 16 * tile_of(u) + lr;
        if (wave + kPolicyWaves * u >= nt || n >= N) continue;
        const float b = bias[n];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 4 * lg + r;
          const float v = last ? acc[u][r] + b : elu(acc[u][r] + b);
          dst[row * kPolicyPitch + n] = v;
          if (last && q.out && row < nr) q.out[(r0 + row) * q.ldo + n] = v;
        }
      }
    }
    __syncthreads();
    cur ^= 1;
  }

  // Sampling (as zk_sample_g32): a 32-lane group per row, lane k on component
  // k; the row's logp terms added in component order by its first lane.
  if (blockIdx.y != 0 || !p.sample) return;
  const int A = p.A;
  if (t < A) {
    s_ls[t] = p.log_std[t];
    s_sdv[t] = expf(s_ls[t]);
  }
  __syncthreads();
  const int g = t / 32, k = t % 32;
  const long long r = r0 + g;
  float term = 0.f;
  if (g < nr && k < A) {
    const float mu = act[cur][g * kPolicyPitch + k];
    const float a = mu + s_sdv[k] * p.eps[r * p.lde + k];
    p.action[r * p.lda + k] = a;
    const float d = (a - mu) / s_sdv[k];
    term = -0.5f * d * d - s_ls[k] - kLogSqrt2Pi;
  }
  s_term[t] = term;
  __syncthreads();
  if (k == 0 && g < nr) {
    float lp = 0.f;
    for (int j = 0; j < A; ++j) lp += s_term[g * 32 + j];
    p.logp[r] = lp;
  }
}

// One float4 of the packed weights per thread (the layout is described with
// PolicyPackArgs). The segment is found by comparing against every
// segment's start with constant indices, so the arguments stay in scalar
// registers.
__device__ void policy_pack_body(const PolicyPackArgs& a) {
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= a.nq) return;
  long long src = 0, dst = 0, q0 = 0;
  int ldw = 0, N = 0, K = 0, kc = 1;
#pragma unroll
  for (int s = 0; s < kPolicyPackSegs; ++s)
    if (s < a.nseg && i >= a.seg[s].q0) {
      src = a.seg[s].src;
      dst = a.seg[s].dst;
      q0 = a.seg[s].q0;
      ldw = a.seg[s].ldw;
      N = a.seg[s].N;
      K = a.seg[s].K;
      kc = a.seg[s].kc;
    }
  const long long j = i - q0;
  const int lane = (int)(j & 63);
  const long long b = j >> 6;
  const int n = 16 * (int)(b / kc) + (lane & 15);
  const int k = 16 * (int)(b % kc) + 4 * (lane >> 4);
  float4 v = {0.f, 0.f, 0.f, 0.f};
  if (n < N && k < K) {
    // k < K <= ldw with k and ldw multiples of 4: the float4 stays in the row.
    v = *reinterpret_cast<const float4*>(a.params + src + (long long)n * ldw + k);
    if (k + 1 >= K) v.y = 0.f;
    if (k + 2 >= K) v.z = 0.f;
    if (k + 3 >= K) v.w = 0.f;
  }
  *reinterpret_cast<float4*>(a.dst + dst + 4 * j) = v;
}

}  // namespace zk

// Held to eight waves per SIMD (two 16-wave blocks per CU, at most 64 VGPRs).
extern "C" __global__ __launch_bounds__(zk::kPolicyThreads) __attribute__((amdgpu_waves_per_eu(8)))
void zk_policy(zk::PolicyArgs p) {
  zk::policy_body(p);
}

extern "C" __global__ __launch_bounds__(zk::kThreads) void zk_policy_pack(zk::PolicyPackArgs a) {
  zk::policy_pack_body(a);
}
