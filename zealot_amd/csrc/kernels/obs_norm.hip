// obs_norm.hip — the running observation normaliser on the device
// (Normalizer and PendingNorm, zealot-rl/src/ppo.rs:104-206).
//
// State: float[2 * dim + 1] = mean[dim], m2[dim], count. The reference folds
// one observation at a time (Welford); here a batch of rows is cut into
// chunks of kNormChunkRows, each chunk's mean and sum of squared deviations
// are taken two-pass in a fixed order (zk_norm_stats), and the chunks are
// merged with the parallel-Welford (Chan) update that Normalizer::commit uses:
// contiguous runs of chunks in row order, then the state with the runs in
// order (zk_norm_merge). mean and m2 therefore agree
// with the one-at-a-time fold to fp32 rounding, not bit for bit; count
// follows the reference exactly (see count_add_ones). zk_norm_commit and
// zk_norm_apply repeat the reference's operation order and are bit-exact.
#pragma once
#include "common.hip"

namespace zk {

// `c + 1.0f` applied n times in f32, as the reference's per-observation
// `count += 1.0` does: exact while the count stays at or below 2^24, where
// the f32 spacing reaches 2 and the increment stops (ties to even).
__device__ __forceinline__ float count_add_ones(float c, long long n) {
  const float kExact = 16777216.0f;  // 2^24
  if (n <= 0) return c;
  if (c >= 0.0f && c <= kExact && c == floorf(c)) {
    if ((double)c + (double)n <= (double)kExact) return (float)((double)c + (double)n);
    c = kExact;  // reached after kExact - c increments; stuck from here on
    return c;
  }
  // Non-integer or larger counts (only from a restored state): step until
  // the increment no longer changes the value.
  for (long long i = 0; i < n; ++i) {
    const float c2 = c + 1.0f;
    if (c2 == c) break;
    c = c2;
  }
  return c;
}

// Normalizer::new (ppo.rs:141-148) or an empty PendingNorm.
__device__ void norm_set_body(const NormArgs& p) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i > 2 * p.dim) return;
  const float prior = p.unit_prior ? 1.0f : 0.0f;
  p.state[i] = i < p.dim ? 0.0f : prior;
}

// Normalizer::normalize (ppo.rs:198-205), rows [blockIdx.x * rows_per_block,
// ...): var = max(m2 / count, 1e-8), out = clamp((x - mean) / sqrt(var), -5, 5)
// with correctly rounded division and square root. For dim <= 256 a pass
// covers 256 / dim whole rows, each thread one fixed column. Dynamic LDS:
// 2 * dim floats (mean, sd).
__device__ void norm_apply_body(const NormArgs& p) {
  extern __shared__ float s_norm[];
  float* s_mean = s_norm;
  float* s_sd = s_norm + p.dim;
  const int t = threadIdx.x;
  const float count = p.state[2 * p.dim];
  for (int c = t; c < p.dim; c += kThreads) {
    s_mean[c] = p.state[c];
    const float var = fmaxf(p.state[p.dim + c] / count, 1e-8f);
    s_sd[c] = sqrtf(var);
  }
  __syncthreads();
  const long long r0 = (long long)blockIdx.x * p.rows_per_block;
  const long long r1 = min(p.rows, r0 + p.rows_per_block);
  if (p.dim <= kThreads) {
    const int g = kThreads / p.dim;  // rows per pass
    const int rr = t / p.dim, c = t - rr * p.dim;
    if (rr >= g) return;
    const float mu = s_mean[c], sd = s_sd[c];
    constexpr int U = 4;
    for (long long r = r0 + rr; r < r1; r += (long long)U * g) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const long long ru = r + (long long)u * g;
        v[u] = ru < r1 ? p.x[ru * p.ldx + c] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const long long ru = r + (long long)u * g;
        if (ru < r1) p.out[ru * p.ldo + c] = clampf((v[u] - mu) / sd, -5.0f, 5.0f);
      }
    }
  } else {
    for (long long r = r0; r < r1; ++r)
      for (int c = t; c < p.dim; c += kThreads)
        p.out[r * p.ldo + c] = clampf((p.x[r * p.ldx + c] - s_mean[c]) / s_sd[c], -5.0f, 5.0f);
  }
}

// Per-chunk statistics: block (chunk k, 64 columns); 4 row lanes of 64
// threads take rows r = lane, lane + 4, ... of the chunk. Pass 1 sums, the
// four lane sums are added in lane order, mean = sum / n; pass 2 does the
// same for (x - mean)^2. part[(2k) * dim + c] = mean, part[(2k + 1) * dim + c] = M2.
__device__ void norm_stats_body(const NormArgs& p) {
  __shared__ float red[4][64];
  __shared__ float s_mean[64];
  const int t = threadIdx.x, cl = t & 63, lane = t >> 6;
  const int c = blockIdx.y * 64 + cl;
  const int k = blockIdx.x;
  const long long r0 = (long long)k * kNormChunkRows;
  const long long r1 = min(p.rows, r0 + kNormChunkRows);
  const float n = (float)(r1 - r0);
  const bool live = c < p.dim;
  float s = 0.0f;
  if (live) {
    constexpr int U = 8;
    for (long long r = r0 + lane; r < r1; r += 4 * U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = r + 4 * u < r1 ? p.x[(r + 4 * u) * p.ldx + c] : 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (r + 4 * u < r1) s += v[u];
    }
  }
  red[lane][cl] = s;
  __syncthreads();
  if (lane == 0) s_mean[cl] = (((red[0][cl] + red[1][cl]) + red[2][cl]) + red[3][cl]) / n;
  __syncthreads();
  const float mu = s_mean[cl];
  float q = 0.0f;
  if (live) {
    constexpr int U = 8;
    for (long long r = r0 + lane; r < r1; r += 4 * U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = r + 4 * u < r1 ? p.x[(r + 4 * u) * p.ldx + c] : 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (r + 4 * u < r1) {
          const float d = v[u] - mu;
          q += d * d;
        }
    }
  }
  __syncthreads();
  red[lane][cl] = q;
  __syncthreads();
  if (lane == 0 && live) {
    p.part[(long long)(2 * k) * p.dim + c] = mu;
    p.part[(long long)(2 * k + 1) * p.dim + c] = ((red[0][cl] + red[1][cl]) + red[2][cl]) + red[3][cl];
  }
}

// Chan merge of (n2, m_b, q_b) into (n1, mean, m2), in Normalizer::commit's
// operation order (ppo.rs:186-190); an empty left side takes the right one.
__device__ __forceinline__ void chan_merge(float& n1, float& mean, float& m2, float n2, float mb,
                                           float qb) {
  if (n2 == 0.0f) return;
  if (n1 == 0.0f) {
    n1 = n2;
    mean = mb;
    m2 = qb;
    return;
  }
  const float tot = n1 + n2;
  const float d = mb - mean;
  mean += d * n2 / tot;
  m2 += qb + d * d * n1 * n2 / tot;
  n1 = tot;
}

// Fold the chunks into the state (one block). Each column has T threads
// (T = the largest power of two <= 1024 / dim, at most 32); thread j merges
// the j-th contiguous run of chunks in row order, then the column's first
// thread merges the state with the T runs in order. The order is fixed, so
// the result is the same on every run.
__device__ void norm_merge_body(const NormArgs& p) {
  __shared__ float s_part[kNormFoldThreads][3];
  const int t = threadIdx.x;
  int T = 1;
  while (T < 32 && 2 * T * p.dim <= kNormFoldThreads) T *= 2;
  const int per = (p.nchunks + T - 1) / T;
  const float count0 = p.state[2 * p.dim];
  const int cols_per_pass = kNormFoldThreads / T;
  for (int c0 = 0; c0 < p.dim; c0 += cols_per_pass) {
    const int c = c0 + t / T, j = t % T;
    float n = 0.0f, mean = 0.0f, m2 = 0.0f;
    if (c < p.dim) {
      const int k1 = min(p.nchunks, (j + 1) * per);
      for (int k = j * per; k < k1; ++k) {
        const long long r0 = (long long)k * kNormChunkRows;
        const float n2 = (float)(min(p.rows, r0 + kNormChunkRows) - r0);
        chan_merge(n, mean, m2, n2, p.part[(long long)(2 * k) * p.dim + c],
                   p.part[(long long)(2 * k + 1) * p.dim + c]);
      }
    }
    s_part[t][0] = n;
    s_part[t][1] = mean;
    s_part[t][2] = m2;
    __syncthreads();
    if (c < p.dim && j == 0) {
      float n1 = count0, sm = p.state[c], sq = p.state[p.dim + c];
      for (int i = 0; i < T; ++i) chan_merge(n1, sm, sq, s_part[t + i][0], s_part[t + i][1], s_part[t + i][2]);
      p.state[c] = sm;
      p.state[p.dim + c] = sq;
    }
    __syncthreads();
  }
  if (t == 0) p.state[2 * p.dim] = count_add_ones(count0, p.rows);  // count0 read by all above
}

// Normalizer::commit (ppo.rs:179-195): merge the pending state, then empty it.
__device__ void norm_commit_body(const NormArgs& p) {
  const int t = threadIdx.x;
  const float n2 = p.pending[2 * p.dim];
  if (n2 == 0.0f) return;  // uniform: nothing pending
  const float n1 = p.state[2 * p.dim];
  const float tot = n1 + n2;
  for (int c = t; c < p.dim; c += kNormFoldThreads) {
    const float d = p.pending[c] - p.state[c];
    p.state[c] += d * n2 / tot;
    p.state[p.dim + c] += p.pending[p.dim + c] + d * d * n1 * n2 / tot;
    p.pending[c] = 0.0f;
    p.pending[p.dim + c] = 0.0f;
  }
  __syncthreads();  // every thread has read both counts
  if (t == 0) {
    p.state[2 * p.dim] = tot;
    p.pending[2 * p.dim] = 0.0f;
  }
}

}  // namespace zk

extern "C" __global__ __launch_bounds__(256) void zk_norm_set(zk::NormArgs p) { zk::norm_set_body(p); }
extern "C" __global__ __launch_bounds__(256) void zk_norm_apply(zk::NormArgs p) { zk::norm_apply_body(p); }
extern "C" __global__ __launch_bounds__(256) void zk_norm_stats(zk::NormArgs p) { zk::norm_stats_body(p); }
extern "C" __global__ __launch_bounds__(zk::kNormFoldThreads) void zk_norm_merge(zk::NormArgs p) {
  zk::norm_merge_body(p);
}
extern "C" __global__ __launch_bounds__(zk::kNormFoldThreads) void zk_norm_commit(zk::NormArgs p) {
  zk::norm_commit_body(p);
}
