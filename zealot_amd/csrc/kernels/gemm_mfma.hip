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
// each LDS orientation makes those reads bank-conflict free. A workgroup is
// WM x WN wave64s; each wave owns TM x TN 16x16 accumulator tiles. K is walked
// in BK-wide k-tiles, double-buffered in LDS with the next k-tile's global
// loads in flight during the MFMAs. BK = 32 makes every K-contiguous row
// segment a full 128-byte line.
//
// Split-K: grid.z slices the k-tiles; each slice writes a dense partial
// [M x N] at C + z*split_stride and zk_splitk_reduce sums the slices in fixed
// order (deterministic, no atomics). Blocks of n-tile 0 can also emit the row
// sums of A per slice (the bias gradient of a weight-gradient GEMM).
#pragma once
#include "common.hip"

namespace zk {

// One operand tile of NT threads: EXT rows/cols along M (or N) by BK along K.
template <int EXT, bool KC, int BK, int NT>
struct Tile {
  // Row length in LDS. K-contiguous rows get +4 floats so 16 rows read at one
  // k hit distinct banks; the other orientation needs LD = 16 or 48 (mod 64)
  // so the four 16-lane k-groups of one read land in disjoint bank windows.
  static constexpr int LD =
      KC ? (BK + 4) : ((EXT % 64 == 16 || EXT % 64 == 48) ? EXT : EXT + 16);
  static constexpr int SIZE = KC ? EXT * LD : BK * LD;
  static constexpr int ELEMS = EXT * BK;
  static constexpr int NV = (ELEMS / 4 + NT - 1) / NT;
  static constexpr int NS = (ELEMS + NT - 1) / NT;
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
        const int i = t + j * NT;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < ELEMS / 4) {
          if (KC) {
            const int row = i / (BK / 4), kq = (i % (BK / 4)) * 4;
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
        const int i = t + j * NT;
        float v = 0.f;
        if (i < ELEMS) {
          if (KC) {
            const int e = e0 + i / BK, k = k0 + i % BK;
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
        const int i = t + j * NT;
        if (i < ELEMS / 4) {
          float4 v = make_float4(r[4 * j], r[4 * j + 1], r[4 * j + 2], r[4 * j + 3]);
          if (KC)
            *reinterpret_cast<float4*>(s + (i / (BK / 4)) * LD + (i % (BK / 4)) * 4) = v;
          else
            *reinterpret_cast<float4*>(s + (i / (EXT / 4)) * LD + (i % (EXT / 4)) * 4) = v;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int i = t + j * NT;
        if (i < ELEMS) {
          if (KC)
            s[(i / BK) * LD + i % BK] = r[j];
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

// KG > 1 splits every staged k-tile between KG groups of WM x WN waves (group
// g runs k-steps [g, g+1) * BK/4/KG); the groups' accumulators are added in
// LDS in group order before the epilogue, so a tile gets KG times the waves
// without any global split-K partials.
template <bool AK, bool BKC, int BM, int BN, int BK, int WM, int WN, int KG = 1>
__device__ __forceinline__ void gemm_body(const GemmArgs& p) {
  constexpr int NT = 64 * WM * WN * KG;
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  static_assert(TM >= 1 && TN >= 1 && TM * WM * 16 == BM && TN * WN * 16 == BN, "wave tiling");
  static_assert(BK % (4 * KG) == 0, "k-steps of 4 per group");
  static_assert(KG == 1 || KG == 2, "one LDS exchange round");
  constexpr int RSG = NT / BM >= 1 ? NT / BM : 1;  // threads per A row in the row sums
  using TA = Tile<BM, AK, BK, NT>;
  using TB = Tile<BN, BKC, BK, NT>;
  constexpr int SMEM = 2 * (TA::SIZE + TB::SIZE);
  static_assert(KG == 1 || SMEM >= BM * BN, "LDS holds one group's accumulator tile");
  static_assert(SMEM >= NT, "LDS holds one float per thread for the row sums");
  // One allocation: [A buf 0][A buf 1][B buf 0][B buf 1], reused after the
  // k-loop for the row-sum and k-group exchanges.
  __shared__ float smem[SMEM];
  auto sA = [&](int b) { return smem + b * TA::SIZE; };
  auto sB = [&](int b) { return smem + 2 * TA::SIZE + b * TB::SIZE; };

  if (p.guard && *p.guard == 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave_all = tid >> 6;
  const int kg = wave_all / (WM * WN), wave = wave_all % (WM * WN);
  const int wm = wave % WM, wn = wave / WM;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  const int KT = (p.K + BK - 1) / BK;
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
  const bool rs_on = rowsum && tid < BM * RSG;

  if (kt0 < kt1) {
    ta.load(p.A, p.lda, m0, p.M, kt0 * BK, p.K, p.permA, vA);
    tb.load(p.B, p.ldb, n0, p.N, kt0 * BK, p.K, p.permB, vB);
    ta.store(sA(0), vA);
    tb.store(sB(0), vB);
  }
  __syncthreads();

  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) {
      ta.load(p.A, p.lda, m0, p.M, (kt + 1) * BK, p.K, p.permA, vA);
      tb.load(p.B, p.ldb, n0, p.N, (kt + 1) * BK, p.K, p.permB, vB);
    }
    const float* as = sA(cur);
    const float* bs = sB(cur);
#pragma unroll
    for (int s = kg * (BK / 4 / KG); s < (kg + 1) * (BK / 4 / KG); ++s) {
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
    if (rs_on) {
      for (int kk = rs_g; kk < BK; kk += RSG) rs += TA::at(as, rs_m, kk);
    }
    if (more) {
      ta.store(sA(cur ^ 1), vA);
      tb.store(sB(cur ^ 1), vB);
    }
    __syncthreads();
  }

  if (rowsum) {
    float* red = smem;  // free after the final barrier
    red[tid] = rs_on ? rs : 0.f;
    __syncthreads();
    if (tid < BM) {
      float tot = 0.f;
      for (int g = 0; g < RSG; ++g) tot += red[g * BM + tid];
      if (m0 + tid < p.M) p.rowsumA[(long long)blockIdx.z * p.M + m0 + tid] = tot;
    }
    __syncthreads();
  }

  if constexpr (KG > 1) {
    // Group 1 hands its accumulators to group 0 through LDS (free after the
    // k-loop and the row-sum barrier).
    float* xch = smem;
    if (kg == 1) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) xch[(((wave * TM + i) * TN + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (kg != 0) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[i][j][r] = acc[i][j][r] + xch[(((wave * TM + i) * TN + j) * 4 + r) * 64 + lane];
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

// out[(i / cols) * ldo + i % cols] = sum_z part[z*mn + i], rowout likewise.
// A block is 256 / lanes elements (float4 quads of the matrix, or single
// row sums) x `lanes` split lanes: lane l adds slices l, l+lanes, ... in
// order (independent loads, so many are in flight per thread), then the
// lanes are combined by a fixed tree in LDS. The order is fixed, so the
// result is deterministic. Blocks past the matrix part reduce the row sums.
__device__ __forceinline__ void splitk_reduce_body(const SplitReduceArgs& p) {
  __shared__ float4 red[256];
  if (p.guard && *p.guard == 0) return;
  const int SL = p.lanes;
  const int QB = 256 / SL;
  const int t = threadIdx.x;
  const int e = t % QB, l = t / QB;
  const long long nq = (p.mn + 3) / 4;
  const long long nqb = (nq + QB - 1) / QB;  // blocks of the matrix part
  const bool matrix = (long long)blockIdx.x < nqb;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  long long idx;
  if (matrix) {
    idx = (long long)blockIdx.x * QB + e;  // quad index
    if (idx < nq) {
      const long long i0 = 4 * idx;
      if ((p.mn & 3) == 0) {
#pragma unroll 4
        for (int z = l; z < p.splits; z += SL) {
          const float4 v = *reinterpret_cast<const float4*>(p.part + (long long)z * p.mn + i0);
          acc.x += v.x;
          acc.y += v.y;
          acc.z += v.z;
          acc.w += v.w;
        }
      } else {
        for (int z = l; z < p.splits; z += SL) {
          const float* b = p.part + (long long)z * p.mn + i0;
          acc.x += b[0];
          if (i0 + 1 < p.mn) acc.y += b[1];
          if (i0 + 2 < p.mn) acc.z += b[2];
          if (i0 + 3 < p.mn) acc.w += b[3];
        }
      }
    }
  } else {
    if (!p.rowpart) return;  // uniform over the block
    idx = ((long long)blockIdx.x - nqb) * QB + e;  // row index
    if (idx < p.rows) {
#pragma unroll 4
      for (int z = l; z < p.splits; z += SL) acc.x += p.rowpart[(long long)z * p.rows + idx];
    }
  }
  red[t] = acc;
  __syncthreads();
  for (int st = SL >> 1; st > 0; st >>= 1) {
    if (l < st) {
      const float4 v = red[t + st * QB];
      float4 a = red[t];
      a.x += v.x;
      a.y += v.y;
      a.z += v.z;
      a.w += v.w;
      red[t] = a;
    }
    __syncthreads();
  }
  if (l != 0) return;
  const float4 s = red[e];
  if (matrix) {
    if (idx >= nq) return;
    const float o[4] = {s.x, s.y, s.z, s.w};
    for (int c = 0; c < 4; ++c) {
      const long long i = 4 * idx + c;
      if (i < p.mn) p.out[(i / p.cols) * p.ldo + i % p.cols] = o[c];
    }
  } else if (idx < p.rows) {
    p.rowout[idx] = s.x;
  }
}

}  // namespace zk

#define ZK_GEMM(NAME, AK, BKC, BM, BN, BK, WM, WN, KG)                                   \
  extern "C" __global__ __launch_bounds__(64 * WM * WN * KG) void NAME(zk::GemmArgs p) { \
    zk::gemm_body<AK, BKC, BM, BN, BK, WM, WN, KG>(p);                                   \
  }

// Naming: a{k,m} = A K- or M-contiguous, b{k,n} = B K- or N-contiguous,
// then BMxBNxBK, the wave grid WMxWN and (k2) two k-groups per tile.
ZK_GEMM(zk_gemm_ak_bk_64x128x16_w22, true, true, 64, 128, 16, 2, 2, 1)
ZK_GEMM(zk_gemm_ak_bk_96x128x32_w24, true, true, 96, 128, 32, 2, 4, 1)
ZK_GEMM(zk_gemm_ak_bk_96x128x16_w24, true, true, 96, 128, 16, 2, 4, 1)
ZK_GEMM(zk_gemm_ak_bk_96x128x32_w22k2, true, true, 96, 128, 32, 2, 2, 2)
ZK_GEMM(zk_gemm_ak_bk_128x32x16_w41, true, true, 128, 32, 16, 4, 1, 1)
ZK_GEMM(zk_gemm_ak_bk_96x32x32_w21, true, true, 96, 32, 32, 2, 1, 1)
ZK_GEMM(zk_gemm_ak_bk_256x16x16_w41, true, true, 256, 16, 16, 4, 1, 1)
ZK_GEMM(zk_gemm_ak_bn_64x128x16_w22, true, false, 64, 128, 16, 2, 2, 1)
ZK_GEMM(zk_gemm_ak_bn_96x128x32_w24, true, false, 96, 128, 32, 2, 4, 1)
ZK_GEMM(zk_gemm_ak_bn_96x128x16_w24, true, false, 96, 128, 16, 2, 4, 1)
ZK_GEMM(zk_gemm_ak_bn_96x128x32_w22k2, true, false, 96, 128, 32, 2, 2, 2)
ZK_GEMM(zk_gemm_am_bn_64x128x16_w22, false, false, 64, 128, 16, 2, 2, 1)
ZK_GEMM(zk_gemm_am_bn_64x128x16_w24, false, false, 64, 128, 16, 2, 4, 1)
ZK_GEMM(zk_gemm_am_bn_64x128x32_w24, false, false, 64, 128, 32, 2, 4, 1)
ZK_GEMM(zk_gemm_am_bn_64x128x32_w22k2, false, false, 64, 128, 32, 2, 2, 2)
ZK_GEMM(zk_gemm_am_bn_128x128x16_w24, false, false, 128, 128, 16, 2, 4, 1)
ZK_GEMM(zk_gemm_am_bn_128x128x32_w22k2, false, false, 128, 128, 32, 2, 2, 2)
ZK_GEMM(zk_gemm_am_bn_64x64x16_w22, false, false, 64, 64, 16, 2, 2, 1)
ZK_GEMM(zk_gemm_am_bn_32x128x16_w14, false, false, 32, 128, 16, 1, 4, 1)
ZK_GEMM(zk_gemm_am_bk_64x128x16_w22, false, true, 64, 128, 16, 2, 2, 1)

extern "C" __global__ __launch_bounds__(256) void zk_splitk_reduce(zk::SplitReduceArgs p) {
  zk::splitk_reduce_body(p);
}
