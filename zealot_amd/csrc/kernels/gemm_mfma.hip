// gemm_mfma.hip — fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x4f32).
//
// C[M x N] = A[M x K] . B[K x N] with fused epilogues. Replaces the cuTile
// kernels gemm_tf32 / gemm_splitk_tf32 / gemm_bias_act_tf32 / reduce_splitk
// (src/biped/cutile_gemm.rs:175-268,315-330) but computes in full fp32, not tf32.
//
// Operand storage: A is either K-contiguous (row m at A + m*lda) or
// M-contiguous (row k at A + k*lda); B is either K-contiguous (row n at
// B + n*ldb) or N-contiguous (row k at B + k*ldb). Each operand tile is staged
// in LDS in its global orientation (float4 global loads -> ds_write_b128) and
// fed to the MFMA with one ds_read_b32 per lane per k-step; the row padding of
// each LDS orientation makes those reads bank-conflict free. A 256-thread
// workgroup is 4 wave64s in a WM x WN grid; each wave owns TM x TN 16x16
// accumulator tiles. K is walked in 16-wide k-tiles, double-buffered in LDS
// with the next k-tile's global loads in flight during the MFMAs.
//
// Split-K: grid.z slices the k-tiles; each slice writes a dense partial
// [M x N] at C + z*split_stride and zk_splitk_reduce sums the slices in fixed
// order (deterministic, no atomics). Blocks of n-tile 0 can also emit the row
// sums of A per slice (the bias gradient of a weight-gradient GEMM).
#pragma once
#include "common.hip"

namespace zk {

constexpr int kBK = 16;

// One operand tile: EXT rows/cols along M (or N) by kBK along K.
template <int EXT, bool KC>
struct Tile {
  static constexpr int LD = KC ? (kBK + 4) : (EXT + 16);
  static constexpr int SIZE = KC ? EXT * LD : kBK * LD;
  static constexpr int ELEMS = EXT * kBK;
  static constexpr int NV = (ELEMS / 4 + kThreads - 1) / kThreads;
  static constexpr int NS = (ELEMS + kThreads - 1) / kThreads;
  static constexpr int NR = (4 * NV > NS) ? 4 * NV : NS;
  float r[NR];

  // Global -> registers. `perm` remaps the storage row (the EXT index when
  // K-contiguous, the k index otherwise). Out-of-range elements load as 0.
  __device__ __forceinline__ void load(const float* __restrict__ base, int ld, int e0, int etot,
                                       int k0, int K, const int* __restrict__ perm, bool vec) {
    const int t = threadIdx.x;
    if (vec) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int i = t + j * kThreads;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < ELEMS / 4) {
          if (KC) {
            const int row = i / (kBK / 4), kq = (i % (kBK / 4)) * 4;
            const int e = e0 + row, k = k0 + kq;
            if (e < etot && k < K) {
              const int sr = perm ? perm[e] : e;
              v = *reinterpret_cast<const float4*>(base + (long long)sr * ld + k);
              if (k + 1 >= K) v.y = 0.f;
              if (k + 2 >= K) v.z = 0.f;
              if (k + 3 >= K) v.w = 0.f;
            }
          } else {
            const int kk = i / (EXT / 4), c4 = (i % (EXT / 4)) * 4;
            const int k = k0 + kk, e = e0 + c4;
            if (k < K && e < etot) {
              const int sr = perm ? perm[k] : k;
              v = *reinterpret_cast<const float4*>(base + (long long)sr * ld + e);
              if (e + 1 >= etot) v.y = 0.f;
              if (e + 2 >= etot) v.z = 0.f;
              if (e + 3 >= etot) v.w = 0.f;
            }
          }
        }
        r[4 * j + 0] = v.x;
        r[4 * j + 1] = v.y;
        r[4 * j + 2] = v.z;
        r[4 * j + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int i = t + j * kThreads;
        float v = 0.f;
        if (i < ELEMS) {
          if (KC) {
            const int e = e0 + i / kBK, k = k0 + i % kBK;
            if (e < etot && k < K) v = base[(long long)(perm ? perm[e] : e) * ld + k];
          } else {
            const int k = k0 + i / EXT, e = e0 + i % EXT;
            if (k < K && e < etot) v = base[(long long)(perm ? perm[k] : k) * ld + e];
          }
        }
        r[j] = v;
      }
    }
  }

  // Registers -> LDS buffer.
  __device__ __forceinline__ void store(float* __restrict__ s, bool vec) const {
    const int t = threadIdx.x;
    if (vec) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int i = t + j * kThreads;
        if (i < ELEMS / 4) {
          float4 v = make_float4(r[4 * j], r[4 * j + 1], r[4 * j + 2], r[4 * j + 3]);
          if (KC)
            *reinterpret_cast<float4*>(s + (i / (kBK / 4)) * LD + (i % (kBK / 4)) * 4) = v;
          else
            *reinterpret_cast<float4*>(s + (i / (EXT / 4)) * LD + (i % (EXT / 4)) * 4) = v;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int i = t + j * kThreads;
        if (i < ELEMS) {
          if (KC)
            s[(i / kBK) * LD + i % kBK] = r[j];
          else
            s[(i / EXT) * LD + i % EXT] = r[j];
        }
      }
    }
  }

  // Element (e, k) of a staged tile.
  __device__ __forceinline__ static float at(const float* s, int e, int k) {
    return KC ? s[e * LD + k] : s[k * LD + e];
  }
};

template <bool AK, bool BKC, int BM, int BN, int WM, int WN>
__device__ __forceinline__ void gemm_body(const GemmArgs& p) {
  static_assert(WM * WN == kThreads / 64, "4 waves per workgroup");
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 16x16 MFMA tile");
  constexpr int RSG = kThreads / BM;  // row-sum groups (threads per A row)
  static_assert(RSG >= 1 && kBK % RSG == 0, "row-sum split");
  using TA = Tile<BM, AK>;
  using TB = Tile<BN, BKC>;
  __shared__ float sA[2][TA::SIZE];
  __shared__ float sB[2][TB::SIZE];

  if (p.guard && *p.guard == 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  const int KT = (p.K + kBK - 1) / kBK;
  const int kt0 = blockIdx.z * p.kt_per_split;
  const int kt1 = min(KT, kt0 + p.kt_per_split);
  const bool rowsum = p.rowsumA != nullptr && blockIdx.y == 0;
  const bool vA = p.vecA != 0, vB = p.vecB != 0;

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  TA ta;
  TB tb;
  float rs = 0.f;
  const int rs_m = tid % BM, rs_g = tid / BM;

  if (kt0 < kt1) {
    ta.load(p.A, p.lda, m0, p.M, kt0 * kBK, p.K, p.permA, vA);
    tb.load(p.B, p.ldb, n0, p.N, kt0 * kBK, p.K, p.permB, vB);
    ta.store(sA[0], vA);
    tb.store(sB[0], vB);
  }
  __syncthreads();

  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) {
      ta.load(p.A, p.lda, m0, p.M, (kt + 1) * kBK, p.K, p.permA, vA);
      tb.load(p.B, p.ldb, n0, p.N, (kt + 1) * kBK, p.K, p.permB, vB);
    }
    const float* as = sA[cur];
    const float* bs = sB[cur];
#pragma unroll
    for (int s = 0; s < kBK / 4; ++s) {
      const int kk = 4 * s + lg;
      float af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = TA::at(as, (wm * TM + i) * 16 + lr, kk);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = TB::at(bs, (wn * TN + j) * 16 + lr, kk);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (rowsum) {
#pragma unroll
      for (int j = 0; j < kBK / RSG; ++j) rs += TA::at(as, rs_m, rs_g * (kBK / RSG) + j);
    }
    if (more) {
      ta.store(sA[cur ^ 1], vA);
      tb.store(sB[cur ^ 1], vB);
    }
    __syncthreads();
  }

  if (rowsum) {
    float* red = sA[0];  // free after the final barrier
    red[tid] = rs;
    __syncthreads();
    if (tid < BM) {
      float tot = 0.f;
#pragma unroll
      for (int g = 0; g < RSG; ++g) tot += red[g * BM + tid];
      if (m0 + tid < p.M) p.rowsumA[(long long)blockIdx.z * p.M + m0 + tid] = tot;
    }
  }

  float* C = p.C + (long long)blockIdx.z * p.split_stride;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + (wn * TN + j) * 16 + lr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + (wm * TM + i) * 16 + lg * 4 + r;
        if (m < p.M && n < p.N) {
          float v = acc[i][j][r];
          if (p.epi == kEpiBiasN) {
            v = v + p.bias[n];
            if (p.act) v = elu(v);
          } else if (p.epi == kEpiBiasM) {
            v = v + p.bias[(long long)m * p.bias_stride];
            if (p.act) v = elu(v);
          } else if (p.epi == kEpiEluGrad) {
            v = v * elu_grad_from_act(p.Y[(long long)m * p.ldy + n]);
          }
          C[(long long)m * p.ldc + n] = v;
        }
      }
    }
  }
}


// out[(i / cols) * ldo + i % cols] = sum_z part[z*mn + i] (z ascending);
// rowout likewise. One thread per output element; the grid covers mn + rows.
__device__ __forceinline__ void splitk_reduce_body(const SplitReduceArgs& p) {
  if (p.guard && *p.guard == 0) return;
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i < p.mn) {
    float s = 0.f;
    for (int z = 0; z < p.splits; ++z) s += p.part[(long long)z * p.mn + i];
    p.out[(i / p.cols) * p.ldo + i % p.cols] = s;
  } else if (p.rowpart && i < p.mn + p.rows) {
    const int r = (int)(i - p.mn);
    float s = 0.f;
    for (int z = 0; z < p.splits; ++z) s += p.rowpart[(long long)z * p.rows + r];
    p.rowout[r] = s;
  }
}

}  // namespace zk

#define ZK_GEMM(NAME, AK, BKC, BM, BN, WM, WN)                           \
  extern "C" __global__ __launch_bounds__(256) void NAME(zk::GemmArgs p) { \
    zk::gemm_body<AK, BKC, BM, BN, WM, WN>(p);                           \
  }

// Naming: a{k,m} = A K- or M-contiguous, b{k,n} = B K- or N-contiguous.
ZK_GEMM(zk_gemm_ak_bk_64x128, true, true, 64, 128, 2, 2)
ZK_GEMM(zk_gemm_ak_bk_128x32, true, true, 128, 32, 4, 1)
ZK_GEMM(zk_gemm_ak_bk_256x16, true, true, 256, 16, 4, 1)
ZK_GEMM(zk_gemm_ak_bn_64x128, true, false, 64, 128, 2, 2)
ZK_GEMM(zk_gemm_am_bn_64x128, false, false, 64, 128, 2, 2)
ZK_GEMM(zk_gemm_am_bk_64x128, false, true, 64, 128, 2, 2)

extern "C" __global__ __launch_bounds__(256) void zk_splitk_reduce(zk::SplitReduceArgs p) {
  zk::splitk_reduce_body(p);
}
