// gemm_mfma.hip — fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x4f32).
//
// C[M x N] = A[M x K] . B[K x N] with fused epilogues. Replaces the cuTile
// kernels gemm_tf32 / gemm_splitk_tf32 / gemm_bias_act_tf32 / reduce_splitk
// (src/biped/cutile_gemm.rs:175-268,315-330) but computes in full fp32, not tf32.
//
// Operand storage: A is either K-contiguous (row m at A + m*lda) or
// M-contiguous (row k at A + k*lda); B is either K-contiguous (row n at
// B + n*ldb) or N-contiguous (row k at B + k*ldb). Each operand tile is staged
// in LDS in its global orientation (float4 global loads -> ds_write_b128). A
// workgroup is WM x WN wave64s; each wave owns TM x TN 16x16 accumulator
// tiles. K is walked in BK-wide k-tiles, double-buffered in LDS, with the
// global loads two k-tiles ahead in registers (see gemm_body). BK = 32 makes
// every K-contiguous row segment a full 128-byte line.
//
// Reduction-index assignment. v_mfma_f32_16x16x4f32 takes A[i][s] from lane
// i + 16 s and B[s][j] from lane j + 16 s. Within each 16-wide chunk q of a
// k-tile, lane group s of MFMA step c carries k = 16 q + 4 s + c in both
// operands (any bijection gives the same sum), so a lane's four k values of
// a chunk are consecutive: a K-contiguous tile feeds four MFMAs with one
// ds_read_b128, the other orientation with four ds_read_b32. LDS is read as
// two half-waves of 32 lanes over 32 banks; the row lengths below make both
// kinds of read conflict-free: BK + 4 (K-contiguous, 8 lanes of 16 rows per
// b128 pass land on 8 disjoint 4-bank groups) and EXT + 4 (the rows k and
// k + 4 of one half-wave are 16 banks apart). That bank model is the one the
// SQ_LDS_BANK_CONFLICT counters of the earlier row-per-lane-group layout fit.
//
// Split-K: grid.z slices the k-tiles; each slice writes a dense partial
// [M x N] at C + z*split_stride and zk_splitk_reduce sums the slices in fixed
// order (deterministic, no atomics). Blocks of n-tile 0 can also emit the row
// sums of A per slice (the bias gradient of a weight-gradient GEMM).
#pragma once
#include "common.hip"

namespace zk {

// One operand tile of NT threads: EXT rows/cols along M (or N) by BK along K.
//
// Global loads are issued unconditionally from clamped, always-valid
// addresses and every bounds / padding mask is applied when the registers are
// written to LDS, one iteration later: nothing between the load and the store
// needs the loaded values, so the loads stay in flight during a k-tile's
// MFMAs. Storage rows gathered through `perm` are resolved once per block for
// a K-contiguous operand (its rows do not change along K) and one k-tile
// ahead of the loads for the other orientation. EXACT tiles are for problems
// whose M, N and K are multiples of the tile (the host checks): no clamps and
// no masks, which leaves the k-loop about 40 % fewer non-MFMA instructions.
template <int EXT, bool KC, int BK, int NT, bool VEC, bool EXACT = false>
struct Tile {
  // Row length in LDS (see the file header): conflict-free fragment reads
  // with 16-byte aligned rows for the ds_write_b128 stores.
  static constexpr int LD = KC ? (BK + 4) : (EXT + 4);
  static constexpr int SIZE = KC ? EXT * LD : BK * LD;
  static constexpr int ELEMS = EXT * BK;
  static constexpr int NQ = ELEMS / 4;            // float4 quads per tile
  static constexpr int NV = (NQ + NT - 1) / NT;   // quads per thread
  static constexpr int NS = (ELEMS + NT - 1) / NT;  // scalars per thread
  static constexpr int QR = KC ? BK / 4 : EXT / 4;  // quads per stored row
  static constexpr int ROWS = KC ? EXT : BK;         // stored rows
  // Stored row of float4 quad i (its column is quad i % QR). With 4 or 8
  // quads per row, a 16-lane pass of a ds_write_b128 would cover 2-4
  // consecutive rows whose bank windows overlap at these row lengths; the
  // rows of one pass are spread QR apart instead, which places them in
  // disjoint bank windows. Eight consecutive lanes still read 128
  // contiguous bytes of one row from global memory.
  __device__ __forceinline__ static int row_of(int i) {
    if constexpr (QR < 16 && 16 % QR == 0 && ROWS % 16 == 0) {
      const int p = i / 16;
      return 16 * (p / QR) + p % QR + ((i % 16) / QR) * QR;
    } else {
      return i / QR;
    }
  }
  float4 v[VEC ? NV : 1];
  float s[VEC ? 1 : NS];
  // Vector path, per quad: KC -> storage row pointer (perm resolved, row
  // clamped); other orientation -> column offset and the perm'd storage row
  // of the k-tile to load next.
  const float* rp[NV];
  int col[NV];
  int pk[NV];
  bool ok[NV];  // quad inside the tile's EXT range (and i < NQ)

  const float* base;
  const int* perm;
  int ld, e0, etot, K;

  __device__ __forceinline__ void init(const float* __restrict__ b, int ld_, int e0_, int etot_,
                                       int K_, const int* __restrict__ perm_) {
    base = b;
    ld = ld_;
    e0 = e0_;
    etot = etot_;
    K = K_;
    perm = perm_;
    if (!VEC) return;
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = t + j * NT;
      const int iq = (NQ % NT == 0 || i < NQ) ? i : 0;
      if (KC) {
        const int e = e0 + row_of(iq);
        ok[j] = (NQ % NT == 0 || i < NQ) && e < etot;
        const int ec = min(e, etot - 1);
        const int sr = perm ? perm[ec] : ec;
        rp[j] = base + (long long)sr * ld;
      } else {
        const int e = e0 + (iq % QR) * 4;
        ok[j] = (NQ % NT == 0 || i < NQ) && e < etot;
        col[j] = min(e, ((etot + 3) & ~3) - 4);
      }
    }
  }

  // Other orientation with a gather: storage rows of the k-tile at k0.
  __device__ __forceinline__ void fetch_rows(int k0) {
    if (KC || !VEC || !perm) return;
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = t + j * NT;
      const int iq = (NQ % NT == 0 || i < NQ) ? i : 0;
      pk[j] = perm[min(k0 + row_of(iq), K - 1)];
    }
  }

  // Global -> registers for the k-tile at k0 (no masking here).
  __device__ __forceinline__ void load(int k0) {
    const int t = threadIdx.x;
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int i = t + j * NT;
        const int iq = (NQ % NT == 0 || i < NQ) ? i : 0;
        if (KC) {
          const int k = EXACT ? k0 + (iq % QR) * 4 : min(k0 + (iq % QR) * 4, ((K + 3) & ~3) - 4);
          v[j] = *reinterpret_cast<const float4*>(rp[j] + k);
        } else {
          const int kc = EXACT ? k0 + row_of(iq) : min(k0 + row_of(iq), K - 1);
          const int sr = perm ? pk[j] : kc;
          v[j] = *reinterpret_cast<const float4*>(base + (long long)sr * ld + col[j]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int i = t + j * NT;
        const int ic = (ELEMS % NT == 0 || i < ELEMS) ? i : 0;
        int e, k;
        if (KC) {
          e = e0 + ic / BK;
          k = k0 + ic % BK;
        } else {
          k = k0 + ic / EXT;
          e = e0 + ic % EXT;
        }
        const int ec = min(e, etot - 1), kc = min(k, K - 1);
        const long long sr = KC ? (perm ? perm[ec] : ec) : (perm ? perm[kc] : kc);
        s[j] = base[sr * ld + (KC ? kc : ec)];
      }
    }
  }

  // Registers -> LDS buffer, zeroing everything outside [0, etot) x [0, K).
  // A k-tile that lies wholly inside the matrix (the common case) is stored
  // without masks.
  __device__ __forceinline__ void store(float* __restrict__ sm, int k0) const {
    const int t = threadIdx.x;
    if constexpr (VEC) {
      const bool full = EXACT || (e0 + EXT <= etot && k0 + BK <= K);
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int i = t + j * NT;
        if (NQ % NT != 0 && i >= NQ) continue;
        float4 x = v[j];
        if (full) {  // row row_of(i), quad i % QR in either orientation
          *reinterpret_cast<float4*>(sm + row_of(i) * LD + (i % QR) * 4) = x;
          continue;
        }
        if (KC) {
          const int kq = (i % QR) * 4, k = k0 + kq;
          const bool good = ok[j] && k < K;
          x.x = good ? x.x : 0.f;
          x.y = (good && k + 1 < K) ? x.y : 0.f;
          x.z = (good && k + 2 < K) ? x.z : 0.f;
          x.w = (good && k + 3 < K) ? x.w : 0.f;
          *reinterpret_cast<float4*>(sm + row_of(i) * LD + kq) = x;
        } else {
          const int kk = row_of(i), c4 = (i % QR) * 4;
          const int e = e0 + c4;
          const bool good = ok[j] && k0 + kk < K;
          x.x = good ? x.x : 0.f;
          x.y = (good && e + 1 < etot) ? x.y : 0.f;
          x.z = (good && e + 2 < etot) ? x.z : 0.f;
          x.w = (good && e + 3 < etot) ? x.w : 0.f;
          *reinterpret_cast<float4*>(sm + kk * LD + c4) = x;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int i = t + j * NT;
        if (ELEMS % NT != 0 && i >= ELEMS) continue;
        int e, k, off;
        if (KC) {
          e = e0 + i / BK;
          k = k0 + i % BK;
          off = (i / BK) * LD + i % BK;
        } else {
          k = k0 + i / EXT;
          e = e0 + i % EXT;
          off = (i / EXT) * LD + i % EXT;
        }
        sm[off] = (e < etot && k < K) ? s[j] : 0.f;
      }
    }
  }

  // Element (e, k) of a staged tile.
  __device__ __forceinline__ static float at(const float* sm, int e, int k) {
    return KC ? sm[e * LD + k] : sm[k * LD + e];
  }

  // MFMA operand fragment of chunk q for lane group g: elements
  // (e, 16 q + 4 g + c), c = 0..3.
  __device__ __forceinline__ static float4 frag(const float* sm, int e, int q, int g) {
    if constexpr (KC) {
      return *reinterpret_cast<const float4*>(sm + e * LD + 16 * q + 4 * g);
    } else {
      const float* x = sm + (16 * q + 4 * g) * LD + e;
      return float4{x[0], x[LD], x[2 * LD], x[3 * LD]};
    }
  }
};

// Tile (mt, nt) and z index (problem x split-K slice) of this block.
// Workgroups reach the 8 XCDs round robin by linear id, and every XCD has its
// own L2, so blocks that read the same rows should sit on one XCD at the same
// time. With a multiple of 8 z slices (the split-K weight gradients) all tiles
// of a slice go to one XCD, slice after slice; otherwise, with a multiple of 8
// tiles, every XCD gets a contiguous run of tiles of its slice, column tile
// fastest (the column tiles that read one A row block together). Both are
// bijections of the launch grid.
struct BlockTile {
  int mt, nt, z;
};
// Tile of the block with linear dispatch index g (x fastest, then y, then z)
// in a gx x ntl x nz grid.
__device__ __forceinline__ BlockTile block_tile_of(int g, int gx, int ntl, int nz) {
  const int ntiles = gx * ntl;
  if (nz % 8 == 0) {
    const int k = g / 8;
    const int t = k % ntiles;
    return {t / ntl, t % ntl, g % 8 + 8 * (k / ntiles)};
  }
  const int b = g % ntiles;
  if (ntiles % 8 == 0) {
    const int t = (b % 8) * (ntiles / 8) + b / 8;
    return {t / ntl, t % ntl, g / ntiles};
  }
  return {b % gx, b / gx, g / ntiles};
}
// Problem and tile of block g of a tiled GemmBatch launch (z = the split-K
// slice within the problem).
__device__ __forceinline__ BlockTile batch_tile(const GemmBatch& b, int g, int& prob) {
  prob = b.count > 1 && g >= b.blk0[1] ? 1 : 0;
  return block_tile_of(g - b.blk0[prob], b.gx[prob], b.gy[prob], b.gz[prob]);
}

// LDS floats of one gemm_body instantiation: both operand tiles, double
// buffered.
template <bool AK, bool BKC, int BM, int BN, int BK, int WM, int WN, bool VEC, bool EXACT = false>
constexpr int gemm_smem_floats() {
  return 2 * (Tile<BM, AK, BK, 64 * WM * WN, VEC, EXACT>::SIZE +
              Tile<BN, BKC, BK, 64 * WM * WN, VEC, EXACT>::SIZE);
}

// LDS_OUT: the epilogue writes the whole BM x BN tile (no bounds tests;
// entries outside C come from zero operands) into the LDS array `cl` with
// row pitch p.ldc instead of to p.C; `cl` may overlap `smem` (it is written
// after the k-loop's last barrier).
template <bool AK, bool BKC, int BM, int BN, int BK, int WM, int WN, bool VEC,
          bool YPRE = false, bool EXACT = false, bool LDS_OUT = false>
__device__ __forceinline__ void gemm_body(float* __restrict__ smem, const GemmArgs& p, int split,
                                          int mt, int nt, float* __restrict__ cl = nullptr) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  static_assert(TM >= 1 && TN >= 1 && TM * WM * 16 == BM && TN * WN * 16 == BN, "wave tiling");
  static_assert(BK % 16 == 0, "16-wide chunks");
  constexpr int RSG = NT / BM >= 1 ? NT / BM : 1;  // threads per A row in the row sums
  using TA = Tile<BM, AK, BK, NT, VEC, EXACT>;
  using TB = Tile<BN, BKC, BK, NT, VEC, EXACT>;
  static_assert(gemm_smem_floats<AK, BKC, BM, BN, BK, WM, WN, VEC, EXACT>() >= NT,
                "LDS holds one float per thread for the row sums");
  // smem (the caller's LDS, gemm_smem_floats of it, 16-byte aligned):
  // [A buf 0][A buf 1][B buf 0][B buf 1], reused after the k-loop for the
  // row-sum exchange.
  auto sA = [&](int b) { return smem + b * TA::SIZE; };
  auto sB = [&](int b) { return smem + 2 * TA::SIZE + b * TB::SIZE; };

  if (p.guard && *p.guard == 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = mt * BM, n0 = nt * BN;
  if (m0 >= p.M || n0 >= p.N || split >= p.nsplit) return;  // outside this problem (uniform)
  const int KT = (p.K + BK - 1) / BK;
  const int kt0 = split * p.kt_per_split;
  const int kt1 = min(KT, kt0 + p.kt_per_split);
  const bool rowsum = p.rowsumA != nullptr && nt == 0;

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  TA ta;
  TB tb;
  ta.init(p.A, p.lda, m0, p.M, p.K, p.permA);
  tb.init(p.B, p.ldb, n0, p.N, p.K, p.permB);
  float rs = 0.f;
  const int rs_m = tid % BM, rs_g = tid / BM;
  const bool rs_on = rowsum && tid < BM * RSG;

  // Column bias of the batch-major forward epilogue, read before the k-loop
  // so that its latency is hidden behind the MFMAs.
  float bpre[TN];
  if (p.epi == kEpiBiasN) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + (wn * TN + j) * 16 + lr;
      bpre[j] = n < p.N ? p.bias[n] : 0.f;
    }
  }

  // Pipeline. Registers hold the global loads of k-tile t + 1 while the MFMAs
  // of k-tile t run; they are written to the free LDS buffer at the start of
  // iteration t, and the loads of k-tile t + 2 are issued right after. The
  // single barrier of an iteration sits before the group's last 16-wide
  // chunk: the fragments of that chunk are read before it, and the first
  // chunk of k-tile t + 1 is read after it while the last chunk's MFMAs run,
  // so no wave waits on an LDS read right after the barrier.
  //   LDS buffer (t + 1) & 1 is written in iteration t: its previous contents
  //   (k-tile t - 1) were last read before the barrier of iteration t - 1.
  //   Its reads happen after the barrier of iteration t.
  if (kt0 < kt1) {
    ta.fetch_rows(kt0 * BK);
    tb.fetch_rows(kt0 * BK);
    ta.load(kt0 * BK);
    tb.load(kt0 * BK);
    ta.store(sA(0), kt0 * BK);
    tb.store(sB(0), kt0 * BK);
    if (kt0 + 1 < kt1) {
      ta.fetch_rows((kt0 + 1) * BK);
      tb.fetch_rows((kt0 + 1) * BK);
      ta.load((kt0 + 1) * BK);
      tb.load((kt0 + 1) * BK);
      if (kt0 + 2 < kt1) {
        ta.fetch_rows((kt0 + 2) * BK);
        tb.fetch_rows((kt0 + 2) * BK);
      }
    }
  }
  __syncthreads();

  // YPRE variants (data gradients): the ELU' operand is read into registers
  // at the start of the last k-tile (which has no tile loads left to issue),
  // so its latency overlaps the last MFMAs instead of the epilogue waiting
  // for it.
  const bool elu_grad = YPRE && p.epi == kEpiEluGrad;
  // Staged epilogue (exact-fit data gradients): the tile goes through LDS so
  // that each thread reads the ELU' operand and stores dL/dz as whole float4
  // row segments (the layer-1 backward 234 -> 229 us per launch; the forward
  // and the weight-gradient partials measured no faster, so they keep the
  // direct stores). The host picks exact-fit forms only for float4-aligned
  // C and Y rows.
  constexpr bool STAGED = EXACT && YPRE && !LDS_OUT;
  constexpr int SQ = BN / 4;        // float4 quads per tile row
  constexpr int SRP = NT / SQ;      // rows per staged pass
  constexpr int SPASS = BM / SRP;   // passes
  constexpr int SPITCH = BN + 4;
  static_assert(!STAGED || (NT % SQ == 0 && BM % SRP == 0 &&
                            BM * SPITCH <= gemm_smem_floats<AK, BKC, BM, BN, BK, WM, WN, VEC, EXACT>()),
                "staged epilogue layout");
  float4 yq[STAGED && YPRE ? SPASS : 1];
  float ypre[YPRE && !STAGED ? TM : 1][YPRE && !STAGED ? TN : 1][4];
  auto prefetch_y = [&]() {
    if constexpr (STAGED) {
#pragma unroll
      for (int ps = 0; ps < SPASS; ++ps) {
        const int ml = tid / SQ + ps * SRP;
        yq[ps] = *reinterpret_cast<const float4*>(p.Y + (long long)(m0 + ml) * p.ldy + n0 + 4 * (tid % SQ));
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + (wn * TN + j) * 16 + lr;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + (wm * TM + i) * 16 + lg * 4 + r;
          if constexpr (YPRE && !STAGED) ypre[i][j][r] = (m < p.M && n < p.N) ? p.Y[(long long)m * p.ldy + n] : 0.f;
        }
      }
  };

  // 16-wide chunks per k-tile.
  constexpr int QPG = BK / 16;
  struct Frags {
    float4 a[TM], b[TN];
  };
  auto read_chunk = [&](Frags& f, const float* as, const float* bs, int qi) {
    const int q = qi;
#pragma unroll
    for (int i = 0; i < TM; ++i) f.a[i] = TA::frag(as, (wm * TM + i) * 16 + lr, q, lg);
#pragma unroll
    for (int j = 0; j < TN; ++j) f.b[j] = TB::frag(bs, (wn * TN + j) * 16 + lr, q, lg);
  };
  auto mma_chunk = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i].x, f.b[j].x, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i].y, f.b[j].y, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i].z, f.b[j].z, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i].w, f.b[j].w, acc[i][j], 0, 0, 0);
      }
  };
  // One iteration; `first` holds chunk 0 of k-tile kt on entry (its MFMAs
  // run before the barrier) and receives chunk 0 of k-tile kt + 1 after it.
  // With a single chunk per group nothing is left to run after the barrier:
  // the next iteration's LDS stores and global loads are issued while that
  // read is in flight.
  Frags fr[QPG];
  auto iteration = [&](int kt, Frags& first) {
    const int cur = (kt - kt0) & 1;
    if (kt + 1 < kt1) {
      ta.store(sA(cur ^ 1), (kt + 1) * BK);
      tb.store(sB(cur ^ 1), (kt + 1) * BK);
    }
    if (kt + 2 < kt1) {
      ta.load((kt + 2) * BK);
      tb.load((kt + 2) * BK);
      if (kt + 3 < kt1) {
        ta.fetch_rows((kt + 3) * BK);
        tb.fetch_rows((kt + 3) * BK);
      }
    }
    const float* as = sA(cur);
    const float* bs = sB(cur);
#pragma unroll
    for (int qi = 1; qi < QPG; ++qi) read_chunk(fr[qi], as, bs, qi);
    mma_chunk(first);
#pragma unroll
    for (int qi = 1; qi + 1 < QPG; ++qi) mma_chunk(fr[qi]);
    if (rs_on) {
      for (int kk = rs_g; kk < BK; kk += RSG) rs += TA::at(as, rs_m, kk);
    }
    __syncthreads();
    if (kt + 1 < kt1) read_chunk(first, sA(cur ^ 1), sB(cur ^ 1), 0);
    if constexpr (QPG > 1) mma_chunk(fr[QPG - 1]);
  };
  // The last k-tile is peeled off the loop, so that the ELU' operand read
  // before it is not held in registers across the loop.
  Frags f0;
  if (kt0 < kt1) read_chunk(f0, sA(0), sB(0), 0);
  for (int kt = kt0; kt + 1 < kt1; ++kt) iteration(kt, f0);
  if (kt0 < kt1) {
    if (elu_grad) prefetch_y();
    iteration(kt1 - 1, f0);
  }

  if (rowsum) {
    float* red = smem;  // free after the final barrier
    red[tid] = rs_on ? rs : 0.f;
    __syncthreads();
    if (tid < BM) {
      float tot = 0.f;
      for (int g = 0; g < RSG; ++g) tot += red[g * BM + tid];
      if (m0 + tid < p.M) p.rowsumA[(long long)split * p.M + m0 + tid] = tot;
    }
    __syncthreads();
  }

  // Epilogue. The kind (and ELU flag) is uniform, so each kind runs its own
  // straight-line element loop; tiles wholly inside C skip the bounds tests.
  float* C = p.C + (long long)split * p.split_stride;
  if constexpr (STAGED) {
    // Every LDS read of the k-loop precedes its last barrier, so the
    // buffers are free: the accumulators go to LDS as they lie, then each
    // thread takes float4 row segments (column quad tid % SQ, rows tid / SQ
    // + SRP * pass) through the epilogue to HBM.
    float* st = smem;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ml = (wm * TM + i) * 16 + lg * 4 + r;
#pragma unroll
        for (int j = 0; j < TN; ++j) st[ml * SPITCH + (wn * TN + j) * 16 + lr] = acc[i][j][r];
      }
    __syncthreads();
    const int cq = tid % SQ;
    const int n = n0 + 4 * cq;
    float4 bq = make_float4(0.f, 0.f, 0.f, 0.f);
    if (p.epi == kEpiBiasN) bq = make_float4(p.bias[n], p.bias[n + 1], p.bias[n + 2], p.bias[n + 3]);
#pragma unroll
    for (int ps = 0; ps < SPASS; ++ps) {
      const int ml = tid / SQ + ps * SRP;
      const long long m = m0 + ml;
      float4 v = *reinterpret_cast<const float4*>(st + ml * SPITCH + 4 * cq);
      if (p.epi == kEpiBiasN) {
        v.x += bq.x;
        v.y += bq.y;
        v.z += bq.z;
        v.w += bq.w;
        if (p.act) {
          v.x = elu(v.x);
          v.y = elu(v.y);
          v.z = elu(v.z);
          v.w = elu(v.w);
        }
      } else if (p.epi == kEpiBiasM) {
        const float bm = p.bias[m * p.bias_stride];
        v.x += bm;
        v.y += bm;
        v.z += bm;
        v.w += bm;
        if (p.act) {
          v.x = elu(v.x);
          v.y = elu(v.y);
          v.z = elu(v.z);
          v.w = elu(v.w);
        }
      } else if (p.epi == kEpiEluGrad) {
        float4 y;
        if constexpr (YPRE)
          y = yq[ps];
        else
          y = *reinterpret_cast<const float4*>(p.Y + m * p.ldy + n);
        v.x *= elu_grad_from_act(y.x);
        v.y *= elu_grad_from_act(y.y);
        v.z *= elu_grad_from_act(y.z);
        v.w *= elu_grad_from_act(y.w);
      }
      *reinterpret_cast<float4*>(C + m * p.ldc + n) = v;
    }
    return;
  }
  const bool full_tile = EXACT || (m0 + BM <= p.M && n0 + BN <= p.N);
  auto emit = [&](auto f) {
    if constexpr (LDS_OUT) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ml = (wm * TM + i) * 16 + lg * 4 + r;
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int nl = (wn * TN + j) * 16 + lr;
            cl[ml * p.ldc + nl] = f(acc[i][j][r], i, j, r, m0 + ml, n0 + nl);
          }
        }
      return;
    }
    auto run = [&](auto full) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + (wm * TM + i) * 16 + lg * 4 + r;
          float* crow = C + (long long)m * p.ldc;
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int n = n0 + (wn * TN + j) * 16 + lr;
            if (decltype(full)::value || (m < p.M && n < p.N)) crow[n] = f(acc[i][j][r], i, j, r, m, n);
          }
        }
    };
    if (full_tile)
      run(std::true_type{});
    else
      run(std::false_type{});
  };
  if (p.epi == kEpiBiasN) {
    if (p.act)
      emit([&](float v, int, int j, int, int, int) { return elu(v + bpre[j]); });
    else
      emit([&](float v, int, int j, int, int, int) { return v + bpre[j]; });
  } else if (p.epi == kEpiBiasM) {
    if (p.act)
      emit([&](float v, int, int, int, int m, int) { return elu(v + p.bias[(long long)m * p.bias_stride]); });
    else
      emit([&](float v, int, int, int, int m, int) { return v + p.bias[(long long)m * p.bias_stride]; });
  } else if (p.epi == kEpiEluGrad) {
    if constexpr (YPRE)
      emit([&](float v, int i, int j, int r, int, int) { return v * elu_grad_from_act(ypre[i][j][r]); });
    else
      emit([&](float v, int, int, int, int m, int n) { return v * elu_grad_from_act(p.Y[(long long)m * p.ldy + n]); });
  } else {
    emit([&](float v, int, int, int, int, int) { return v; });
  }
}

// Small-K form of the A K-contiguous x B N-contiguous product (the
// reference's feature-major gemm_bias_act, src/biped/cutile_gemm.rs:578-625,
// at K <= KP): every global load of the block -- the whole K extent of both
// operand tiles -- is issued in one round, stored to LDS once, and the MFMAs
// then run over the 16-wide chunks from LDS, so the block pays one memory
// latency instead of one per k-tile. A may be read element by element (VA =
// false: rows that are not 16-byte aligned, such as a 123-float stride); B
// is read as float4 rows. Epilogues: store, bias per column (kEpiBiasN) or
// per row (kEpiBiasM), optional ELU. No split-K, row sums or gathers.
template <int BM, int BN, int KP, int WM, int WN, bool VA>
constexpr int gemm_smallk_smem_floats() {
  return Tile<BM, true, KP, 64 * WM * WN, VA>::SIZE + Tile<BN, false, KP, 64 * WM * WN, true>::SIZE;
}
template <int BM, int BN, int KP, int WM, int WN, bool VA>
__device__ __forceinline__ void gemm_smallk_body(float* __restrict__ smem, const GemmArgs& p, int mt,
                                                 int nt) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  static_assert(TM * WM * 16 == BM && TN * WN * 16 == BN && KP % 16 == 0, "small-K tiling");
  using TA = Tile<BM, true, KP, NT, VA>;
  using TB = Tile<BN, false, KP, NT, true>;
  float* sA = smem;
  float* sB = smem + TA::SIZE;
  if (p.guard && *p.guard == 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = mt * BM, n0 = nt * BN;
  if (m0 >= p.M || n0 >= p.N) return;
  TA ta;
  TB tb;
  ta.init(p.A, p.lda, m0, p.M, p.K, nullptr);
  tb.init(p.B, p.ldb, n0, p.N, p.K, nullptr);
  ta.load(0);
  tb.load(0);
  ta.store(sA, 0);  // zero past K and past the matrix edges
  tb.store(sB, 0);
  __syncthreads();
  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int nq = (p.K + 15) / 16;
  float4 fa[TM], fb[TN];
  auto read = [&](int q) {
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = TA::frag(sA, (wm * TM + i) * 16 + lr, q, lg);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[j] = TB::frag(sB, (wn * TN + j) * 16 + lr, q, lg);
  };
  read(0);
  for (int q = 0; q < nq; ++q) {
    float4 a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = fa[i];
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = fb[j];
    if (q + 1 < nq) read(q + 1);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
      }
  }
  const bool full = m0 + BM <= p.M && n0 + BN <= p.N;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + (wm * TM + i) * 16 + lg * 4 + r;
      if (!full && m >= p.M) continue;
      const float bm = p.epi == kEpiBiasM ? p.bias[(long long)m * p.bias_stride] : 0.f;
      float* crow = p.C + (long long)m * p.ldc;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + (wn * TN + j) * 16 + lr;
        if (!full && n >= p.N) continue;
        float v = acc[i][j][r];
        if (p.epi == kEpiBiasN) v += p.bias[n];
        if (p.epi == kEpiBiasM) v += bm;
        if (p.epi != kEpiStore && p.act) v = elu(v);
        crow[n] = v;
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

// All weight and bias gradients of an update step in one launch
// (ReduceAllArgs): block b finds its segment, sums its outputs over the
// segment's slices in the fixed order of splitk_reduce_body (or reads them
// when the tensor is already final), writes them, and writes the fixed-order
// sum of their squares to sq_part[b] — the grad-norm partials of the clip,
// actor segments first.
__device__ __forceinline__ void reduce_all_body(const ReduceAllArgs& a) {
  __shared__ float4 red[kReduceAllThreads];
  __shared__ float sqs[kReduceAllThreads];
  if (a.guard && *a.guard == 0) return;
  int si = 0;
  for (int i = 1; i < a.nseg; ++i)
    if ((int)blockIdx.x >= a.seg[i].blk0) si = i;
  const ReduceSeg& p = a.seg[si];
  const int SL = p.lanes;
  const int QB = kReduceAllThreads / SL;
  const int t = threadIdx.x;
  const int e = t % QB, l = t / QB;
  const int b = (int)blockIdx.x - p.blk0;
  const long long nq = (p.mn + 3) / 4;
  const bool matrix = b < p.nqb;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  long long idx;
  if (matrix) {
    idx = (long long)b * QB + e;
    if (idx < nq) {
      const long long i0 = 4 * idx;
      if (p.part) {
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
            const float* q = p.part + (long long)z * p.mn + i0;
            acc.x += q[0];
            if (i0 + 1 < p.mn) acc.y += q[1];
            if (i0 + 2 < p.mn) acc.z += q[2];
            if (i0 + 3 < p.mn) acc.w += q[3];
          }
        }
      } else if (l == 0) {
        float o[4] = {0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < 4; ++c) {
          const long long i = i0 + c;
          if (i < p.mn) o[c] = p.out[(i / p.cols) * p.ldo + i % p.cols];
        }
        acc = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
  } else {
    idx = (long long)(b - p.nqb) * QB + e;  // row index
    if (idx < p.rows) {
      if (p.rowpart) {
#pragma unroll 4
        for (int z = l; z < p.splits; z += SL) acc.x += p.rowpart[(long long)z * p.rows + idx];
      } else if (l == 0) {
        acc.x = p.rowout[idx];
      }
    }
  }
  red[t] = acc;
  __syncthreads();
  for (int st = SL >> 1; st > 0; st >>= 1) {
    if (l < st) {
      const float4 v = red[t + st * QB];
      float4 x = red[t];
      x.x += v.x;
      x.y += v.y;
      x.z += v.z;
      x.w += v.w;
      red[t] = x;
    }
    __syncthreads();
  }
  float sq = 0.f;
  if (l == 0) {
    const float4 v = red[e];
    if (matrix) {
      if (idx < nq) {
        const float o[4] = {v.x, v.y, v.z, v.w};
        // Row and column of the quad's first element by one division; the
        // next three follow by stepping the column.
        long long r = 4 * idx / p.cols;
        int col = (int)(4 * idx - r * p.cols);
        for (int c = 0; c < 4; ++c) {
          const long long i = 4 * idx + c;
          if (i < p.mn) {
            if (p.part) p.out[r * p.ldo + col] = o[c];
            sq += o[c] * o[c];
          }
          if (++col == p.cols) {
            col = 0;
            ++r;
          }
        }
      }
    } else if (idx < p.rows) {
      if (p.rowpart) p.rowout[idx] = v.x;
      sq = v.x * v.x;
    }
  }
  const float tot = block_sum<kReduceAllThreads>(sq, sqs);
  if (t == 0 && a.sq_part) a.sq_part[blockIdx.x] = tot;
}

}  // namespace zk

#define ZK_GEMM_X(NAME, AK, BKC, BM, BN, BK, WM, WN, VEC, EXACT)                               \
  extern "C" __global__ __launch_bounds__(64 * WM * WN) void NAME(zk::GemmBatch b) {         \
    __shared__ __align__(16) float smem[zk::gemm_smem_floats<AK, BKC, BM, BN, BK, WM, WN, VEC, EXACT>()]; \
    int prob;                                                                                \
    const zk::BlockTile bt = zk::batch_tile(b, (int)blockIdx.x, prob);                       \
    zk::gemm_body<AK, BKC, BM, BN, BK, WM, WN, VEC, false, EXACT>(smem, b.g[prob], bt.z, bt.mt, bt.nt); \
  }
#define ZK_GEMM(NAME, AK, BKC, BM, BN, BK, WM, WN, VEC) \
  ZK_GEMM_X(NAME, AK, BKC, BM, BN, BK, WM, WN, VEC, false)

// Naming: a{k,m} = A K- or M-contiguous, b{k,n} = B K- or N-contiguous,
// then BMxBNxBK, the wave grid WMxWN and (_s) scalar global loads for
// operands that are not 16-byte aligned row by row.
ZK_GEMM(zk_gemm_ak_bk_128x128x32_w24, true, true, 128, 128, 32, 2, 4, true)
ZK_GEMM(zk_gemm_ak_bk_96x128x32_w24, true, true, 96, 128, 32, 2, 4, true)
ZK_GEMM(zk_gemm_ak_bk_64x64x32_w22, true, true, 64, 64, 32, 2, 2, true)
ZK_GEMM(zk_gemm_ak_bk_32x64x32_w12, true, true, 32, 64, 32, 1, 2, true)
ZK_GEMM(zk_gemm_ak_bk_128x32x16_w41, true, true, 128, 32, 16, 4, 1, true)
ZK_GEMM(zk_gemm_ak_bk_256x16x16_w41, true, true, 256, 16, 16, 4, 1, true)
ZK_GEMM(zk_gemm_ak_bn_96x128x32_w24, true, false, 96, 128, 32, 2, 4, true)
ZK_GEMM(zk_gemm_ak_bn_64x64x32_w22, true, false, 64, 64, 32, 2, 2, true)
// Data-gradient variant (ELU' operand prefetched), held to 4 waves per SIMD
// so that two 8-wave blocks stay resident per CU.
extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
void zk_gemm_ak_bn_96x128x32_w24_dg(zk::GemmBatch b) {
  __shared__ __align__(16) float smem[zk::gemm_smem_floats<true, false, 96, 128, 32, 2, 4, true>()];
  int prob;
  const zk::BlockTile bt = zk::batch_tile(b, (int)blockIdx.x, prob);
  zk::gemm_body<true, false, 96, 128, 32, 2, 4, true, true>(smem, b.g[prob], bt.z, bt.mt, bt.nt);
}
extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
void zk_gemm_ak_bn_96x128x32_w24_dg_x(zk::GemmBatch b) {
  __shared__ __align__(16) float smem[zk::gemm_smem_floats<true, false, 96, 128, 32, 2, 4, true, true>()];
  int prob;
  const zk::BlockTile bt = zk::batch_tile(b, (int)blockIdx.x, prob);
  zk::gemm_body<true, false, 96, 128, 32, 2, 4, true, true, true>(smem, b.g[prob], bt.z, bt.mt, bt.nt);
}
// Exact-fit forms (suffix _x) of the update's layer-GEMM variants.
ZK_GEMM_X(zk_gemm_ak_bk_128x128x32_w24_x, true, true, 128, 128, 32, 2, 4, true, true)
ZK_GEMM_X(zk_gemm_ak_bk_96x128x32_w24_x, true, true, 96, 128, 32, 2, 4, true, true)
ZK_GEMM_X(zk_gemm_am_bn_128x128x32_w24_x, false, false, 128, 128, 32, 2, 4, true, true)
ZK_GEMM_X(zk_gemm_am_bn_64x128x32_w24_x, false, false, 64, 128, 32, 2, 4, true, true)
ZK_GEMM(zk_gemm_am_bn_64x128x32_w24, false, false, 64, 128, 32, 2, 4, true)
ZK_GEMM(zk_gemm_am_bn_128x96x32_w42, false, false, 128, 96, 32, 4, 2, true)
ZK_GEMM_X(zk_gemm_am_bn_128x96x32_w42_x, false, false, 128, 96, 32, 4, 2, true, true)
ZK_GEMM(zk_gemm_am_bn_128x64x32_w42, false, false, 128, 64, 32, 4, 2, true)
ZK_GEMM_X(zk_gemm_am_bn_128x64x32_w42_x, false, false, 128, 64, 32, 4, 2, true, true)
ZK_GEMM(zk_gemm_am_bn_128x128x32_w24, false, false, 128, 128, 32, 2, 4, true)
ZK_GEMM(zk_gemm_am_bn_32x128x16_w14, false, false, 32, 128, 16, 1, 4, true)
ZK_GEMM(zk_gemm_am_bk_64x128x16_w22, false, true, 64, 128, 16, 2, 2, true)
ZK_GEMM(zk_gemm_ak_bk_64x128x16_w22_s, true, true, 64, 128, 16, 2, 2, false)
ZK_GEMM(zk_gemm_ak_bn_64x128x16_w22_s, true, false, 64, 128, 16, 2, 2, false)
ZK_GEMM(zk_gemm_ak_bn_64x64x32_w22_s, true, false, 64, 64, 32, 2, 2, false)
ZK_GEMM(zk_gemm_am_bn_64x128x16_w22_s, false, false, 64, 128, 16, 2, 2, false)
ZK_GEMM(zk_gemm_am_bk_64x128x16_w22_s, false, true, 64, 128, 16, 2, 2, false)

// Small-K variants (K <= 128): A element loads (_s) or float4 rows.
#define ZK_GEMM_SMALLK(NAME, BM, BN, WM, WN, VA)                                                 \
  extern "C" __global__ __launch_bounds__(64 * WM * WN) void NAME(zk::GemmBatch b) {            \
    __shared__ __align__(16) float smem[zk::gemm_smallk_smem_floats<BM, BN, 128, WM, WN, VA>()]; \
    int prob;                                                                                   \
    const zk::BlockTile bt = zk::batch_tile(b, (int)blockIdx.x, prob);                          \
    zk::gemm_smallk_body<BM, BN, 128, WM, WN, VA>(smem, b.g[prob], bt.mt, bt.nt);               \
  }
ZK_GEMM_SMALLK(zk_gemm_ak_bn_64x64xk128_w22_s, 64, 64, 2, 2, false)
ZK_GEMM_SMALLK(zk_gemm_ak_bn_64x64xk128_w22, 64, 64, 2, 2, true)
ZK_GEMM_SMALLK(zk_gemm_ak_bn_64x64xk128_w24_s, 64, 64, 2, 4, false)
ZK_GEMM_SMALLK(zk_gemm_ak_bn_64x64xk128_w24, 64, 64, 2, 4, true)

// One layer's backward as one launch (GemmPair): the split-K weight-gradient
// GEMMs of both nets (exact-fit am_bn tiles, blocks [0, w grid)) and their
// data-gradient GEMMs with the ELU' epilogue (exact-fit DBM x 128 ak_bn tiles,
// the blocks after). The two parts read the same dL/dz and write disjoint
// outputs; one grid lets data-gradient tiles start on the CUs that the
// weight-gradient slices leave, instead of a second launch after the first
// one's last block. The parts share one LDS allocation, the larger of the two.
#define ZK_GEMM_BWD(NAME, WBM, DBM)                                                               \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))           \
  void NAME(zk::GemmPair b) {                                                                     \
    constexpr int SW = zk::gemm_smem_floats<false, false, WBM, 128, 32, 2, 4, true, true>();      \
    constexpr int SD = zk::gemm_smem_floats<true, false, DBM, 128, 32, 2, 4, true, true>();       \
    __shared__ __align__(16) float smem[SW > SD ? SW : SD];                                       \
    const int g = (int)blockIdx.x;                                                                 \
    int prob;                                                                                      \
    if (g < b.nw) {                                                                                \
      const zk::BlockTile bt = zk::batch_tile(b.w, g, prob);                                      \
      zk::gemm_body<false, false, WBM, 128, 32, 2, 4, true, false, true>(smem, b.w.g[prob], bt.z,   \
                                                                        bt.mt, bt.nt);             \
    } else {                                                                                       \
      const zk::BlockTile bt = zk::batch_tile(b.d, g - b.nw, prob);                               \
      zk::gemm_body<true, false, DBM, 128, 32, 2, 4, true, true, true>(smem, b.d.g[prob], bt.z,     \
                                                                     bt.mt, bt.nt);                \
    }                                                                                              \
  }
ZK_GEMM_BWD(zk_gemm_bwd_128x128_dg_x, 128, 96)
ZK_GEMM_BWD(zk_gemm_bwd_64x128_dg_x, 64, 96)
ZK_GEMM_BWD(zk_gemm_bwd_128x128_dg128_x, 128, 128)
ZK_GEMM_BWD(zk_gemm_bwd_64x128_dg128_x, 64, 128)
extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
void zk_gemm_ak_bn_128x128x32_w24_dg(zk::GemmBatch b) {
  __shared__ __align__(16) float smem[zk::gemm_smem_floats<true, false, 128, 128, 32, 2, 4, true>()];
  int prob;
  const zk::BlockTile bt = zk::batch_tile(b, (int)blockIdx.x, prob);
  zk::gemm_body<true, false, 128, 128, 32, 2, 4, true, true>(smem, b.g[prob], bt.z, bt.mt, bt.nt);
}
extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
void zk_gemm_ak_bn_128x128x32_w24_dg_x(zk::GemmBatch b) {
  __shared__ __align__(16) float smem[zk::gemm_smem_floats<true, false, 128, 128, 32, 2, 4, true, true>()];
  int prob;
  const zk::BlockTile bt = zk::batch_tile(b, (int)blockIdx.x, prob);
  zk::gemm_body<true, false, 128, 128, 32, 2, 4, true, true, true>(smem, b.g[prob], bt.z, bt.mt, bt.nt);
}

extern "C" __global__ __launch_bounds__(256) void zk_splitk_reduce(zk::SplitReduceArgs p) {
  zk::splitk_reduce_body(p);
}

