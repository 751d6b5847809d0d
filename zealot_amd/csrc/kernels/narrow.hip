// narrow.hip — GEMMs with one dimension <= 32 on CDNA4 matrix cores
// (v_mfma_f32_16x16x4f32): the output heads of the policy and value MLPs.
//
// The tiled kernels of gemm_mfma.hip stage every k-tile through LDS behind a
// barrier; with one dimension of 1..32 there is too little work per tile to
// hide that round trip, and too few tiles to fill 256 CUs. Here each
// wavefront owns whole 16-row strips and keeps its operands in registers: no
// LDS in the k-loop, no barriers, every load of a strip issued up front.
//
// Reduction-index assignment. v_mfma_f32_16x16x4f32 reads A[i][s] from lane
// (i + 16 s) and B[s][j] from lane (j + 16 s) for the four k-slots s of one
// step. Any bijection between (step, slot) and the reduction index gives the
// same sum as long as A and B use the same one, so lane group s at step c of
// the 16-wide chunk k0 carries index k0 + 4 s + c: one float4 load per lane
// feeds four consecutive MFMAs.
//
//   zk_narrow_n*  C[M x N] = A[M x K] . B[N x K]^T (+ bias, ELU), N <= 32
//                 (the forward of an output layer; A rows may be gathered).
//   zk_narrow_k   C[M x N] = A[M x K] . B[K x N] (x ELU'(Y)), K <= 32
//                 (the data gradient through an output layer).
//   zk_narrow_m*  C[M x N] = A^T . B over K rows, A stored [K x M] (M <= 32),
//                 B stored [K x N] (the weight gradient of an output layer):
//                 blockIdx.x slices the rows (fixed-order partials reduced
//                 by zk_splitk_reduce, like split-K), blockIdx.y takes 64
//                 columns; also the row sums of A (the bias gradient).
#pragma once
#include "common.hip"

namespace zk {

// Wavefronts per block of the narrow kernels, and 16-column tiles per block
// of the weight-gradient form.
constexpr int kNarrowWaves = 4;
constexpr int kNarrowMTiles = 4;

// The epilogue shared with the tiled kernels (gemm_mfma.hip).
__device__ __forceinline__ float narrow_epilogue(const GemmArgs& p, float v, int m, int n) {
  if (p.epi == kEpiBiasN) {
    v = v + p.bias[n];
    if (p.act) v = elu(v);
  } else if (p.epi == kEpiBiasM) {
    v = v + p.bias[(long long)m * p.bias_stride];
    if (p.act) v = elu(v);
  } else if (p.epi == kEpiEluGrad) {
    v = v * elu_grad_from_act(p.Y[(long long)m * p.ldy + n]);
  }
  return v;
}

// C = A . B^T, both K-contiguous, N <= 16 * NT. VEC: K % 16 == 0 and both
// operands' rows 16-byte aligned (float4 loads); otherwise element loads
// with the K tail zeroed. K is walked in passes of 128: all loads of a pass
// are issued before its first MFMA, so a strip costs one memory latency per
// pass rather than one per 16-wide chunk.
template <int NT, bool VEC>
__device__ __forceinline__ void narrow_n_body(const GemmArgs& p) {
  constexpr int KC = 8;  // 16-wide chunks per pass
  if (p.guard && *p.guard == 0) return;
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kNarrowWaves + (threadIdx.x >> 6)) * 16;
  if (row0 >= p.M) return;  // uniform over the wavefront
  const int lr = lane & 15, lg = lane >> 4;
  const int m = min(row0 + lr, p.M - 1);
  const long long sr = p.permA ? p.permA[m] : m;
  const float* a = p.A + sr * p.lda;
  const float* b[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) b[t] = p.B + (long long)min(16 * t + lr, p.N - 1) * p.ldb;
  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int K = p.K;
  for (int kp = 0; kp < K; kp += 16 * KC) {
    if constexpr (VEC) {
      float4 av[KC], bv[KC][NT];
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const int k = kp + 16 * j + 4 * lg;
        const bool in = kp + 16 * j < K;  // uniform: K % 16 == 0
        av[j] = in ? *reinterpret_cast<const float4*>(a + k) : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < NT; ++t)
          bv[j][t] = in ? *reinterpret_cast<const float4*>(b[t] + k) : float4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        if (kp + 16 * j < K) {
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].x, bv[j][t].x, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].y, bv[j][t].y, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].z, bv[j][t].z, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].w, bv[j][t].w, acc[t], 0, 0, 0);
          }
        }
      }
    } else {
      for (int k0 = kp; k0 < min(K, kp + 16 * KC); k0 += 16) {
        float av[4], bv[4][NT];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int k = k0 + 4 * lg + c;
          const bool in = k < K;
          av[c] = in ? a[k] : 0.f;
#pragma unroll
          for (int t = 0; t < NT; ++t) bv[c][t] = in ? b[t][k] : 0.f;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int t = 0; t < NT; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[c], bv[c][t], acc[t], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = 16 * t + lr;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int mm = row0 + 4 * lg + r;
      if (mm < p.M && n < p.N) p.C[(long long)mm * p.ldc + n] = narrow_epilogue(p, acc[t][r], mm, n);
    }
  }
}

// C = A . B, A K-contiguous with K <= 32, B N-contiguous ([K x N]). A block's
// wavefronts take 16-row strips; blockIdx.y takes 32 columns (two 16-column
// tiles), so every load of a wavefront (its A strip, both tiles' B columns
// and the ELU' operand of a data gradient) is issued before its MFMAs.
__device__ __forceinline__ void narrow_k_body(const GemmArgs& p) {
  constexpr int NTK = 2;  // 16-column tiles per wavefront
  if (p.guard && *p.guard == 0) return;
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kNarrowWaves + (threadIdx.x >> 6)) * 16;
  if (row0 >= p.M) return;
  const int lr = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.y * (16 * NTK);
  if (n0 >= p.N) return;  // outside this problem of the batch
  const int m = min(row0 + lr, p.M - 1);
  const long long sr = p.permA ? p.permA[m] : m;
  const float* a = p.A + sr * p.lda;
  const int K = p.K;
  const bool elu_grad = p.epi == kEpiEluGrad;
  float av[8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = 16 * j + 4 * lg + c;
      av[4 * j + c] = k < K ? a[k] : 0.f;
    }
  float y[NTK][4], bv[NTK][8];
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    const int n = n0 + 16 * t + lr;
    const bool nin = n < p.N;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int mm = row0 + 4 * lg + r;
      y[t][r] = (elu_grad && nin && mm < p.M) ? p.Y[(long long)mm * p.ldy + n] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = 16 * j + 4 * lg + c;
        bv[t][4 * j + c] = (nin && k < K) ? p.B[(long long)k * p.ldb + n] : 0.f;
      }
  }
  const int nj = K > 16 ? 2 : 1;  // uniform
#pragma unroll
  for (int t = 0; t < NTK; ++t) {
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (j < nj)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[4 * j + c], bv[t][4 * j + c], acc, 0, 0, 0);
    const int nn = n0 + 16 * t + lr;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int mm = row0 + 4 * lg + r;
      if (mm < p.M && nn < p.N) {
        const float v = elu_grad ? acc[r] * elu_grad_from_act(y[t][r]) : narrow_epilogue(p, acc[r], mm, nn);
        p.C[(long long)mm * p.ldc + nn] = v;
      }
    }
  }
}

// C = A^T . B reduced over the rows [z*R, min(K, (z+1)*R)) of slice
// z = blockIdx.x (R = p.kt_per_split, a multiple of 16), for the 64 columns
// n0 = 64 * blockIdx.y; A stored [K x M] with M <= 16 * MT, B stored
// [K x N]; both row-gathered through permA / permB when set. Wavefront w
// takes the 16-row chunks w, w + 4, ... of the slice with all loads of a
// chunk issued first (one row pointer per operand and row, column offsets
// as immediates, out-of-range lanes masked); the four wavefronts'
// accumulators are then added in LDS in wavefront order, so each slice's
// partial is a fixed-order sum. Blocks of column chunk 0 also write the
// slice's row sums of A^T (sums over the rows of each column of A).
template <int MT>
__device__ __forceinline__ void narrow_m_body(const GemmArgs& p) {
  constexpr int NTC = kNarrowMTiles;  // 16-column tiles per block
  constexpr int CH = 1;               // 16-row chunks loaded together
  __shared__ float red[(kNarrowWaves - 1) * MT * NTC * 4 * 64];
  __shared__ float rsred[kNarrowWaves * MT * 64];
  if (p.guard && *p.guard == 0) return;
  // Outside this problem of the batch (uniform over the block).
  if ((int)blockIdx.x >= p.nsplit || (int)blockIdx.y * 16 * NTC >= p.N) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int kb = blockIdx.x * p.kt_per_split;
  const int ke = min(p.K, kb + p.kt_per_split);
  const int n0 = blockIdx.y * (16 * NTC);
  const int ntn = min(NTC, (p.N - n0 + 15) / 16);  // live column tiles (uniform)
  const bool rowsum = p.rowsumA != nullptr && blockIdx.y == 0;
  bool min_[MT], nin[NTC];
#pragma unroll
  for (int i = 0; i < MT; ++i) min_[i] = 16 * i + lr < p.M;
#pragma unroll
  for (int t = 0; t < NTC; ++t) nin[t] = n0 + 16 * t + lr < p.N;
  floatx4 acc[MT][NTC];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NTC; ++t) acc[i][t] = floatx4{0.f, 0.f, 0.f, 0.f};
  float rs[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) rs[i] = 0.f;

  for (int k0 = kb + 16 * wave; k0 < ke; k0 += 16 * kNarrowWaves * CH) {
    float av[CH][4][MT], bv[CH][4][NTC];
#pragma unroll
    for (int h = 0; h < CH; ++h)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = k0 + 16 * kNarrowWaves * h + 4 * lg + c;
        const bool in = k < ke;
        const long long kr = in ? k : kb;
        const long long ra = p.permA ? p.permA[kr] : kr;
        const long long rb = p.permB ? p.permB[kr] : kr;
        const float* arow = p.A + ra * p.lda + lr;
        const float* brow = p.B + rb * p.ldb + n0 + lr;
#pragma unroll
        for (int i = 0; i < MT; ++i) av[h][c][i] = (in && min_[i]) ? arow[16 * i] : 0.f;
#pragma unroll
        for (int t = 0; t < NTC; ++t) bv[h][c][t] = (in && nin[t]) ? brow[16 * t] : 0.f;
      }
#pragma unroll
    for (int h = 0; h < CH; ++h)
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          rs[i] += av[h][c][i];
#pragma unroll
          for (int t = 0; t < NTC; ++t)
            if (t < ntn)
              acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[h][c][i], bv[h][c][t], acc[i][t], 0, 0, 0);
        }
  }

  // Wavefronts 1..3 hand their accumulators to wavefront 0, which adds them
  // in wavefront order.
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int t = 0; t < NTC; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          red[((((wave - 1) * MT + i) * NTC + t) * 4 + r) * 64 + lane] = acc[i][t][r];
  }
#pragma unroll
  for (int i = 0; i < MT; ++i) rsred[(wave * MT + i) * 64 + lane] = rs[i];
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < kNarrowWaves; ++w)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int t = 0; t < NTC; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[i][t][r] = acc[i][t][r] + red[((((w - 1) * MT + i) * NTC + t) * 4 + r) * 64 + lane];

  float* C = p.C + (long long)blockIdx.x * p.split_stride;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NTC; ++t) {
      const int n = n0 + 16 * t + lr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int mm = 16 * i + 4 * lg + r;
        if (t < ntn && mm < p.M && n < p.N)
          C[(long long)mm * p.ldc + n] = narrow_epilogue(p, acc[i][t][r], mm, n);
      }
    }
  if (rowsum && lg == 0) {
    // Column m = 16 i + lr of A: its lane-group partials over the wavefronts,
    // in (wavefront, lane group) order.
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      float tot = 0.f;
      for (int w = 0; w < kNarrowWaves; ++w)
#pragma unroll
        for (int g = 0; g < 4; ++g) tot += rsred[(w * MT + i) * 64 + g * 16 + lr];
      const int mm = 16 * i + lr;
      if (mm < p.M) p.rowsumA[(long long)blockIdx.x * p.M + mm] = tot;
    }
  }
}

}  // namespace zk

// grid.z = problem of the batch (one slice per problem: zper = 1).
#define ZK_NARROW(NAME, BODY)                                                                 \
  extern "C" __global__ __launch_bounds__(64 * zk::kNarrowWaves) void NAME(zk::GemmBatch b) { \
    if ((int)blockIdx.z >= b.count) return;                                                   \
    BODY(b.g[blockIdx.z]);                                                                    \
  }

ZK_NARROW(zk_narrow_n1_v, (zk::narrow_n_body<1, true>))
ZK_NARROW(zk_narrow_n2_v, (zk::narrow_n_body<2, true>))
ZK_NARROW(zk_narrow_n1_s, (zk::narrow_n_body<1, false>))
ZK_NARROW(zk_narrow_n2_s, (zk::narrow_n_body<2, false>))
ZK_NARROW(zk_narrow_k, zk::narrow_k_body)
ZK_NARROW(zk_narrow_m1, zk::narrow_m_body<1>)
ZK_NARROW(zk_narrow_m2, zk::narrow_m_body<2>)
