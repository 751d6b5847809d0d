// runtime.cpp — context, code-object loading, buffers and the stand-alone
// operators of the C ABI (include/zealot_hip.h).
#include <dlfcn.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "internal.hpp"

namespace zl {

const char* const kFixedNames[K_GEMM_BASE] = {
    "zk_splitk_reduce", "zk_actor_loss",  "zk_value_loss", "zk_sumsq",
    "zk_adam",          "zk_epoch_begin", "zk_kl",         "zk_epoch_end",   "zk_gae",
    "zk_adv_norm",      "zk_elu_backward", "zk_row_sum",   "zk_copy_rows",   "zk_sample",
    "zk_clamp",         "zk_reduce_all",  "zk_actor_loss_g64", "zk_head",       "zk_norm_set",
    "zk_norm_apply",
    "zk_norm_stats",    "zk_norm_merge",  "zk_norm_commit", "zk_sample_g32",  "zk_sample_g64",
    "zk_stage",         "zk_sumsq_multi", "zk_clip_scale",  "zk_adam_multi",
    "zk_gemm_bwd_128x128_dg_x", "zk_gemm_bwd_64x128_dg_x", "zk_gemm_bwd_128x128_dg128_x", "zk_gemm_bwd_64x128_dg128_x", "zk_head_fwd", "zk_head_fwd_x",
    "zk_policy",        "zk_transpose",   "zk_policy_pack",
};

// {name, A K-contiguous, B K-contiguous, BM, BN, BK, threads, float4 loads, family}
const GemmKernel kGemmTable[] = {
    {"zk_gemm_ak_bk_96x128x32_w24", true, true, 96, 128, 32, 512, true},
    {"zk_gemm_ak_bk_64x64x32_w22", true, true, 64, 64, 32, 256, true},
    {"zk_gemm_ak_bk_32x64x32_w12", true, true, 32, 64, 32, 128, true},
    {"zk_gemm_ak_bk_128x32x16_w41", true, true, 128, 32, 16, 256, true},
    {"zk_gemm_ak_bk_256x16x16_w41", true, true, 256, 16, 16, 256, true},
    {"zk_gemm_ak_bn_96x128x32_w24", true, false, 96, 128, 32, 512, true},
    {"zk_gemm_ak_bn_96x128x32_w24_dg", true, false, 96, 128, 32, 512, true},
    {"zk_gemm_ak_bk_96x128x32_w24_x", true, true, 96, 128, 32, 512, true},
    {"zk_gemm_ak_bk_128x128x32_w24", true, true, 128, 128, 32, 512, true},
    {"zk_gemm_ak_bk_128x128x32_w24_x", true, true, 128, 128, 32, 512, true},
    {"zk_gemm_ak_bn_96x128x32_w24_dg_x", true, false, 96, 128, 32, 512, true},
    {"zk_gemm_ak_bn_128x128x32_w24_dg", true, false, 128, 128, 32, 512, true},
    {"zk_gemm_ak_bn_128x128x32_w24_dg_x", true, false, 128, 128, 32, 512, true},
    {"zk_gemm_am_bn_128x128x32_w24_x", false, false, 128, 128, 32, 512, true},
    {"zk_gemm_am_bn_64x128x32_w24_x", false, false, 64, 128, 32, 512, true},
    {"zk_gemm_am_bn_64x128x32_w24", false, false, 64, 128, 32, 512, true},
    {"zk_gemm_am_bn_128x128x32_w24", false, false, 128, 128, 32, 512, true},
    {"zk_gemm_am_bn_32x128x16_w14", false, false, 32, 128, 16, 256, true},
    {"zk_gemm_am_bn_128x96x32_w42", false, false, 128, 96, 32, 512, true},
    {"zk_gemm_am_bn_128x96x32_w42_x", false, false, 128, 96, 32, 512, true},
    {"zk_gemm_am_bn_128x64x32_w42", false, false, 128, 64, 32, 512, true},
    {"zk_gemm_am_bn_128x64x32_w42_x", false, false, 128, 64, 32, 512, true},
    {"zk_gemm_am_bk_64x128x16_w22", false, true, 64, 128, 16, 256, true},
    {"zk_gemm_ak_bk_64x128x16_w22_s", true, true, 64, 128, 16, 256, false},
    {"zk_gemm_ak_bn_64x128x16_w22_s", true, false, 64, 128, 16, 256, false},
    {"zk_gemm_am_bn_64x128x16_w22_s", false, false, 64, 128, 16, 256, false},
    {"zk_gemm_am_bk_64x128x16_w22_s", false, true, 64, 128, 16, 256, false},
    {"zk_gemm_ak_bn_64x64x32_w22", true, false, 64, 64, 32, 256, true},
    {"zk_gemm_ak_bn_64x64x32_w22_s", true, false, 64, 64, 32, 256, false},
    {"zk_gemm_ak_bn_64x64xk128_w22_s", true, false, 64, 64, 128, 256, false, G_TILED, true},
    {"zk_gemm_ak_bn_64x64xk128_w22", true, false, 64, 64, 128, 256, true},
    {"zk_gemm_ak_bn_64x64xk128_w24_s", true, false, 64, 64, 128, 512, false, G_TILED, true},
    {"zk_gemm_ak_bn_64x64xk128_w24", true, false, 64, 64, 128, 512, true},
    {"zk_narrow_n1_v", true, true, kNarrowRows, 16, 16, 256, true, G_NARROW_N},
    {"zk_narrow_n2_v", true, true, kNarrowRows, 32, 16, 256, true, G_NARROW_N},
    {"zk_narrow_n1_s", true, true, kNarrowRows, 16, 16, 256, false, G_NARROW_N},
    {"zk_narrow_n2_s", true, true, kNarrowRows, 32, 16, 256, false, G_NARROW_N},
    {"zk_narrow_k", true, false, kNarrowRows, kNarrowKCols, 32, 256, false, G_NARROW_K},
    {"zk_narrow_m1", false, false, 16, kNarrowCols, 16, 256, false, G_NARROW_M},
    {"zk_narrow_m2", false, false, 32, kNarrowCols, 16, 256, false, G_NARROW_M},
};
const int kGemmCount = (int)(sizeof(kGemmTable) / sizeof(kGemmTable[0]));

int kernel_count() { return K_GEMM_BASE + kGemmCount; }

const char* kernel_name(int id) {
  if (id < 0 || id >= kernel_count()) return "?";
  return id < K_GEMM_BASE ? kFixedNames[id] : kGemmTable[id - K_GEMM_BASE].name;
}

static int gemm_id(const char* name) {
  for (int i = 0; i < kGemmCount; ++i)
    if (strcmp(kGemmTable[i].name, name) == 0) return K_GEMM_BASE + i;
  return -1;
}

// Exact-fit twin (name + "_x": no clamps or masks, for M, N and K that are
// multiples of the tile) of a tiled variant, and back; -1 if there is none.
static int exact_form(int kid) {
  const std::string n = std::string(kernel_name(kid)) + "_x";
  return gemm_id(n.c_str());
}
static int inexact_form(int kid) {
  const std::string n = kernel_name(kid);
  if (n.size() < 2 || n.compare(n.size() - 2, 2, "_x") != 0) return kid;
  return gemm_id(n.substr(0, n.size() - 2).c_str());
}

static thread_local std::string g_init_error;

zl_status fail(zl_ctx* c, zl_status s, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  if (c)
    c->err = buf;
  else
    g_init_error = buf;
  return s;
}

zl_status timing_mark(zl_ctx* c, bool stop, int kernel, double flops) {
  // A start mark takes a fresh pair from the pool; a stop mark closes it.
  if (!stop) {
    if (c->ev_used * 2 + 2 > c->ev_pool.size()) {
      for (int i = 0; i < 2; ++i) {
        hipEvent_t e;
        ZL_HIP(c, hipEventCreate(&e));
        c->ev_pool.push_back(e);
      }
    }
    if (c->ev_kernel.size() <= c->ev_used) {
      c->ev_kernel.resize(c->ev_used + 1);
      c->ev_flops.resize(c->ev_used + 1);
      c->ev_shape.resize(c->ev_used + 1);
    }
    c->ev_kernel[c->ev_used] = kernel;
    c->ev_flops[c->ev_used] = flops;
    c->ev_shape[c->ev_used] = c->pending_shape;
    ZL_HIP(c, hipEventRecord(c->ev_pool[c->ev_used * 2], c->stream));
  } else {
    ZL_HIP(c, hipEventRecord(c->ev_pool[c->ev_used * 2 + 1], c->stream));
    c->ev_used += 1;
  }
  return ZL_OK;
}

zl_status ensure_ws(zl_ctx* c, size_t floats) {
  if (floats <= c->ws_floats) return ZL_OK;
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  if (c->ws) ZL_HIP(c, hipFree(c->ws));
  c->ws = nullptr;
  c->ws_floats = 0;
  size_t want = std::max<size_t>(floats, 1 << 20);
  ZL_HIP(c, hipMalloc((void**)&c->ws, want * sizeof(float)));
  c->ws_floats = want;
  return ZL_OK;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Variant choice. The row-major forwards take the largest of 128 x 128,
// 96 x 128, 64 x 64 and 32 x 64 tiles that still gives every CU a
// workgroup; the data gradients 128 x 128 tiles where the rows divide into
// them, else 96 x 128; other A-K-contiguous / B-N-contiguous products (the
// feature-major layers, short-batch data gradients) 96 x 128 on long row
// counts, else 64 x 64; the narrow output layers narrow-N tiles. The weight
// gradients (M x N small, K = rows, split-K) use 128 x 128 tiles for the
// 512- and 256-wide layers, 64 x 128 for the 128-wide one (both with 32-row
// k-tiles, so that the k-loop's barrier sits between two chunks) and
// 32 x 128 for the narrow heads (measured on gfx950 at 24,576 rows).
int pick_gemm(const zl_ctx* c, int M, int N, int K, bool a_kc, bool b_kc, bool vec, int epi,
              bool vec_b) {
  const int lay = layout_of(a_kc, b_kc);
  const bool forced = c && c->force_gemm[lay] >= 0;
  // K <= 128 with B float4-aligned: one round of loads for the whole K
  // extent (the single 4096 x 123 -> 512 feature-major layer, whose weight
  // rows of 123 floats are not float4-aligned).
  if (!forced && c && c->smallk > 0 && lay == L_AK_BN && K > 0 && K <= 128 && vec_b &&
      (epi == zk::kEpiStore || epi == zk::kEpiBiasN || epi == zk::kEpiBiasM) &&
      (!vec || c->smallk > 1))
    return gemm_id(c->smallk_waves == 8 ? (vec ? "zk_gemm_ak_bn_64x64xk128_w24" : "zk_gemm_ak_bn_64x64xk128_w24_s")
                                        : (vec ? "zk_gemm_ak_bn_64x64xk128_w22" : "zk_gemm_ak_bn_64x64xk128_w22_s"));
  if (!forced && (!c || c->narrow)) {
    if (lay == L_AK_BK && N <= 32) {
      const bool v = vec && K % 16 == 0;
      if (N <= 16) return gemm_id(v ? "zk_narrow_n1_v" : "zk_narrow_n1_s");
      return gemm_id(v ? "zk_narrow_n2_v" : "zk_narrow_n2_s");
    }
    if (lay == L_AK_BN && K <= 32) return gemm_id("zk_narrow_k");
    if (lay == L_AM_BN && M <= 32) return gemm_id(M <= 16 ? "zk_narrow_m1" : "zk_narrow_m2");
  }
  if (!vec) {
    if (forced && !kGemmTable[c->force_gemm[lay] - K_GEMM_BASE].vec) return c->force_gemm[lay];
    // Feature-major layers with an odd reduction width (the single
    // 4096-column 123 -> 512 layer: 25.7 -> 20.7 us) take 64 x 64 tiles while
    // 64 x 128 ones would leave CUs with fewer than two workgroups.
    if (lay == L_AK_BN && (long long)cdiv(M, 64) * cdiv(N, 128) < 512) return gemm_id("zk_gemm_ak_bn_64x64x32_w22_s");
    static const char* const kScalar[4] = {
        "zk_gemm_ak_bk_64x128x16_w22_s", "zk_gemm_ak_bn_64x128x16_w22_s",
        "zk_gemm_am_bn_64x128x16_w22_s", "zk_gemm_am_bk_64x128x16_w22_s"};
    return gemm_id(kScalar[lay]);
  }
  if (forced) return c->force_gemm[lay];
  const char* name = nullptr;
  switch (lay) {
    case L_AK_BK:
      if (N <= 16)
        name = "zk_gemm_ak_bk_256x16x16_w41";
      else if (N <= 32)
        name = "zk_gemm_ak_bk_128x32x16_w41";
      else {
        // Largest tile that still gives every CU a workgroup (small-batch
        // forwards such as a 4096-env rollout step), else the smallest.
        // (64 x 64 x 32 ahead of 64 x 128 x 16: its 32-row k-tiles measured
        // faster on the 4,096-row rollout step's 123 -> 512 layer; 128 x 128
        // ahead of 96 x 128: the update's 24,576-row forwards 72.9 -> 69.3 us
        // (123 -> 512) and 114.3 -> 108.2 us (512 -> 256) per pair.)
        static const char* const kFill[4] = {"zk_gemm_ak_bk_128x128x32_w24", "zk_gemm_ak_bk_96x128x32_w24",
                                             "zk_gemm_ak_bk_64x64x32_w22", "zk_gemm_ak_bk_32x64x32_w12"};
        static const int kTile[4][2] = {{128, 128}, {96, 128}, {64, 64}, {32, 64}};
        int pick = 3;
        for (int i = 0; i < 4; ++i)
          if (cdiv(M, kTile[i][0]) * cdiv(N, kTile[i][1]) >= 256) {
            pick = i;
            break;
          }
        name = kFill[pick];
      }
      break;
    case L_AK_BN:
      // Data gradients (ELU' epilogue) take the variant that prefetches the
      // activation operand: 128-row tiles where the rows divide into them
      // (24,576-row layer-1 / layer-2 backward 226.3 -> 224.6 / 71.9 ->
      // 70.7 us), else 96-row tiles. The rest take 96 x 128 tiles on long
      // row counts that give two workgroups per CU, else 64 x 64 (the
      // feature-major 512 x 4096 x 128 layer 17.7 -> 14.8 us, 256 x 4096 x
      // 512 35.6 -> 22.2 us, 8192 x 128 x 256 24.7 -> 15.1 us).
      if (M >= 4096 && epi == zk::kEpiEluGrad)
        name = M % 128 == 0 ? "zk_gemm_ak_bn_128x128x32_w24_dg" : "zk_gemm_ak_bn_96x128x32_w24_dg";
      else if (M >= 4096 && (long long)cdiv(M, 96) * cdiv(N, 128) >= 512)
        name = "zk_gemm_ak_bn_96x128x32_w24";
      else
        name = "zk_gemm_ak_bn_64x64x32_w22";
      break;
    case L_AM_BN:
      // Widths that 128-column tiles would leave partly empty but 96 or 64
      // divide (the trainer nets' input layers: 265 -> 288 padded columns,
      // 64 columns) take tiles that fit them exactly.
      if (M >= 256 && N % 128 != 0 && N % 96 == 0)
        name = "zk_gemm_am_bn_128x96x32_w42";
      else if (M >= 256 && N % 128 != 0 && N % 64 == 0)
        name = "zk_gemm_am_bn_128x64x32_w42";
      else if (M >= 256)
        name = "zk_gemm_am_bn_128x128x32_w24";
      else if (M >= 96)
        name = "zk_gemm_am_bn_64x128x32_w24";
      else
        name = "zk_gemm_am_bn_32x128x16_w14";
      break;
    default:
      name = "zk_gemm_am_bk_64x128x16_w22";
      break;
  }
  (void)K;
  return gemm_id(name);
}

// Rows per slice of a narrow weight-gradient GEMM: a multiple of
// kNarrowSliceQuantum (one round of its wavefronts' two-chunk loads) so that
// slices x column chunks come near the narrow block target.
static int narrow_rows_per_slice(const zl_ctx* c, int N, int K, int epi) {
  const long long full = round_up(std::max(K, 1), 16);
  if (epi != zk::kEpiStore) return (int)full;  // epilogues need the whole sum: one slice
  const long long gy = cdiv(N, kNarrowCols);
  const long long target = std::max<long long>(1, (c ? c->narrow_target : 256) / gy);
  const long long r = round_up(cdiv(K, target), kNarrowSliceQuantum);
  return (int)std::min(r, full);
}

int gemm_splits(const zl_ctx* c, int M, int N, int K, bool a_kc, bool b_kc, int epi, bool vec) {
  const GemmKernel& g = kGemmTable[pick_gemm(c, M, N, K, a_kc, b_kc, vec) - K_GEMM_BASE];
  if (g.kind == G_NARROW_M) return (int)cdiv(std::max(K, 1), narrow_rows_per_slice(c, N, K, epi));
  if (g.kind != G_TILED) return 1;
  if (epi != zk::kEpiStore) return 1;
  const long long tiles = cdiv(M, g.bm) * cdiv(N, g.bn);
  const long long kt = cdiv(K, g.bk);
  long long s;
  if (c && c->force_splits > 0) {
    s = c->force_splits;
  } else {
    // Deep-K, few-tile shapes (the weight gradients, K = batch rows) would
    // leave most CUs idle: slice K so the grid reaches the split-K target
    // (256 = one workgroup per CU: more slices buy no speed in the GEMM at
    // 24,576 rows and cost reduction traffic), keeping at least 8 k-tiles
    // per slice.
    int target = c ? c->splitk_target : 256;
    if (tiles >= target || kt < 16) return 1;
    // Tiles narrower than 128 columns (the odd-width input layers, launched
    // alone) whose slices would run past 16 k-tiles aim at two workgroups
    // per CU (the trainer actor's 256 x 288 input layer: 59.0 -> 46.8 us;
    // the critic's 512 x 64, 12 k-tiles per slice, stays: 24.5 us).
    if (g.bn < 128 && cdiv(kt, cdiv(target, tiles)) > 16) target *= 2;
    s = std::min<long long>(cdiv(target, tiles), std::max<long long>(1, kt / 8));
  }
  s = std::max<long long>(1, std::min(s, kt));
  const long long per = cdiv(kt, s);
  return (int)cdiv(kt, per);
}

size_t gemm_ws_floats(const zl_ctx* c, int M, int N, int K, bool a_kc, bool b_kc, int epi) {
  // Enough for either variant family (operand alignment is known at launch).
  int s = std::max(gemm_splits(c, M, N, K, a_kc, b_kc, epi, true),
                   gemm_splits(c, M, N, K, a_kc, b_kc, epi, false));
  if (s <= 1) return 0;
  return (size_t)s * M * N + (size_t)s * M;
}

static int reduce_lanes(int splits);

zl_status launch_splitk_reduce(zl_ctx* c, zk::SplitReduceArgs& r) {
  const int sl = reduce_lanes(r.splits);
  r.lanes = sl;
  const int per_block = kThreads / sl;
  const long long nqb = cdiv(cdiv(r.mn, 4), per_block);
  const long long nrb = r.rowpart ? cdiv(r.rows, per_block) : 0;
  return launch(c, K_SPLITK_REDUCE, (unsigned)(nqb + nrb), 1, 1, r);
}

// Variant, split-K slicing and tile grid of one GEMM problem.
struct GemmPlan {
  int kid = -1;
  bool vec = false;
  int splits = 1, per = 0;
  unsigned gx = 0, gy = 0;
};

static zl_status plan_gemm(zl_ctx* c, const GemmDesc& d, GemmPlan& P) {
  // float4 row loads need 16-byte aligned rows that cover the padded extent.
  const int a_ext = d.a_kc ? d.K : d.M;
  const int b_ext = d.b_kc ? d.K : d.N;
  const bool va = aligned16(d.A) && d.lda % 4 == 0 && d.lda >= round_up(a_ext, 4);
  const bool vb = aligned16(d.B) && d.ldb % 4 == 0 && d.ldb >= round_up(b_ext, 4);
  P.vec = va && vb;
  const bool plain = !d.rowsum_out && !d.permA && !d.permB && d.splits <= 1;
  P.kid = pick_gemm(c, d.M, d.N, d.K, d.a_kc, d.b_kc, P.vec, d.epi, vb && plain);
  if (P.kid < 0) return fail(c, ZL_ERR_INVALID, "no GEMM variant for this layout");
  const GemmKernel& g = kGemmTable[P.kid - K_GEMM_BASE];
  if (g.a_kc != d.a_kc || g.b_kc != d.b_kc || (g.vec && !P.vec) || (g.need_vec_b && !(vb && plain)))
    return fail(c, ZL_ERR_INVALID, "GEMM variant %s does not match the operand layout", g.name);
  if (strstr(g.name, "xk128") && (d.K > 128 || !plain))
    return fail(c, ZL_ERR_INVALID, "GEMM variant %s takes K <= 128 without split-K, row sums or gathers",
                g.name);
  if (g.kind == G_NARROW_N || g.kind == G_NARROW_K) {
    P.splits = 1;
    P.per = 0;
    P.gx = (unsigned)cdiv(d.M, kNarrowRows);
    P.gy = g.kind == G_NARROW_K ? (unsigned)cdiv(d.N, kNarrowKCols) : 1u;
  } else if (g.kind == G_NARROW_M) {
    P.per = narrow_rows_per_slice(c, d.N, d.K, d.epi);
    P.splits = (int)cdiv(std::max(d.K, 1), P.per);
    P.gx = (unsigned)P.splits;
    P.gy = (unsigned)cdiv(d.N, kNarrowCols);
  } else {
    int splits = d.splits > 0 ? d.splits : gemm_splits(c, d.M, d.N, d.K, d.a_kc, d.b_kc, d.epi, P.vec);
    if (d.epi != zk::kEpiStore) splits = 1;
    const long long kt = cdiv(std::max(d.K, 0), g.bk);
    P.per = (int)std::max<long long>(1, cdiv(kt, splits));
    P.splits = (int)std::max<long long>(1, cdiv(kt, P.per));
    P.gx = (unsigned)cdiv(d.M, g.bm);
    P.gy = (unsigned)cdiv(d.N, g.bn);
    // Every tile and k-tile full: the exact-fit form of the same variant
    // (which may store C and read the ELU' operand as float4 row segments:
    // those rows must be 16-byte aligned, unless C is the split-K scratch).
    const bool c_vec = P.splits > 1 || (aligned16(d.C) && d.ldc % 4 == 0);
    const bool y_vec = d.epi != zk::kEpiEluGrad || (aligned16(d.Y) && d.ldy % 4 == 0);
    if (d.K > 0 && d.M % g.bm == 0 && d.N % g.bn == 0 && d.K % g.bk == 0 && c_vec && y_vec) {
      const int x = exact_form(P.kid);
      if (x >= 0) P.kid = x;
    }
  }
  return ZL_OK;
}

// One grouped launch, planned: its live problems, variant, grid, arguments
// and split-K partial buffers.
struct BatchLaunch {
  const GemmDesc* live[zk::kMaxGemmBatch] = {};
  GemmPlan P[zk::kMaxGemmBatch];
  int nl = 0;
  int kid = -1;
  unsigned gx = 0, gy = 0, gz = 0, threads = 0;
  zk::GemmBatch B{};
  float* part[zk::kMaxGemmBatch] = {};
  double flops = 0.0;
};

// Plans the launch of the problems d[0..n) with a non-empty output. `one` is
// set when they can share a single launch (then L is complete); otherwise
// the caller runs them one by one.
static zl_status plan_batch(zl_ctx* c, const GemmDesc* d, int n, BatchLaunch& L, bool& one) {
  one = false;
  L.nl = 0;
  for (int i = 0; i < n; ++i)
    if (d[i].M > 0 && d[i].N > 0) {
      if (L.nl == zk::kMaxGemmBatch) return fail(c, ZL_ERR_INVALID, "GEMM batch of %d problems", n);
      L.live[L.nl++] = &d[i];
    }
  const int nl = L.nl;
  if (nl == 0) return ZL_OK;
  const GemmDesc* const* live = L.live;
  GemmPlan* P = L.P;
  for (int i = 0; i < nl; ++i) {
    zl_status s = plan_gemm(c, *live[i], P[i]);
    if (s) return s;
  }
  // Narrow kernels size one grid for both problems, so only problems of one
  // shape share such a launch. (Tiled kernels give each problem its own
  // block range, so the actor's and the critic's layer share a launch
  // whatever their shapes.)
  const bool narrow_pair = nl == 2 && kGemmTable[P[0].kid - K_GEMM_BASE].kind != G_TILED &&
                           kGemmTable[P[1].kid - K_GEMM_BASE].kind != G_TILED;
  if (narrow_pair &&
      (live[0]->M != live[1]->M || live[0]->N != live[1]->N || live[0]->K != live[1]->K))
    return ZL_OK;
  // A pair whose members differ only in exact fit runs as one launch of
  // the general form.
  if (nl == 2 && P[0].kid != P[1].kid && inexact_form(P[0].kid) == inexact_form(P[1].kid))
    P[0].kid = P[1].kid = inexact_form(P[0].kid);
  if (nl == 2 && P[0].kid != P[1].kid) {
    // Two narrow problems of one family that differ only in the template
    // width (16 vs 32 columns / rows, float4 vs element loads) share the
    // variant that serves both: the wider, element loads unless both can
    // use float4.
    const GemmKernel& g0 = kGemmTable[P[0].kid - K_GEMM_BASE];
    const GemmKernel& g1 = kGemmTable[P[1].kid - K_GEMM_BASE];
    int shared = -1;
    if (g0.kind == G_NARROW_N && g1.kind == G_NARROW_N) {
      const bool wide = live[0]->N > 16 || live[1]->N > 16;
      const bool v = g0.vec && g1.vec;
      shared = gemm_id(wide ? (v ? "zk_narrow_n2_v" : "zk_narrow_n2_s") : (v ? "zk_narrow_n1_v" : "zk_narrow_n1_s"));
    } else if (g0.kind == G_NARROW_M && g1.kind == G_NARROW_M) {
      shared = gemm_id(live[0]->M > 16 || live[1]->M > 16 ? "zk_narrow_m2" : "zk_narrow_m1");
    }
    if (shared < 0) return ZL_OK;
    P[0].kid = P[1].kid = shared;
  }
  const GemmKernel& g = kGemmTable[P[0].kid - K_GEMM_BASE];
  zk::GemmBatch& B = L.B;
  B = zk::GemmBatch{};
  B.count = nl;
  B.zper = 1;
  unsigned gx = 0, gy = 0;
  double flops = 0.0;
  for (int i = 0; i < nl; ++i) {
    const GemmDesc& q = *live[i];
    zk::GemmArgs& a = B.g[i];
    a.A = q.A;
    a.B = q.B;
    a.bias = q.bias;
    a.Y = q.Y;
    a.permA = q.permA;
    a.permB = q.permB;
    a.guard = q.guard;
    a.M = q.M;
    a.N = q.N;
    a.K = q.K;
    a.lda = q.lda;
    a.ldb = q.ldb;
    a.ldy = q.ldy;
    a.bias_stride = q.bias_stride;
    a.epi = q.epi;
    a.act = q.act;
    a.kt_per_split = P[i].per;
    a.nsplit = P[i].splits;
    a.vecA = P[i].vec;
    a.vecB = P[i].vec;
    L.part[i] = nullptr;
    if (P[i].splits == 1) {
      a.C = q.C;
      a.ldc = q.ldc;
      a.split_stride = 0;
      a.rowsumA = q.rowsum_out;
    } else {
      const size_t mn = (size_t)q.M * q.N;
      const size_t need = (size_t)P[i].splits * mn + (q.rowsum_out ? (size_t)P[i].splits * q.M : 0);
      float* ws = q.ws;
      if (!ws) {
        if (nl > 1) return fail(c, ZL_ERR_INVALID, "batched split-K needs caller scratch");
        zl_status s = ensure_ws(c, need);
        if (s) return s;
        ws = c->ws;
      } else if (need > q.ws_floats) {
        return fail(c, ZL_ERR_INVALID, "split-K scratch too small (%zu < %zu floats)", q.ws_floats,
                    need);
      }
      L.part[i] = ws;
      a.C = ws;
      a.ldc = q.N;
      a.split_stride = (long long)mn;
      a.rowsumA = q.rowsum_out ? ws + (size_t)P[i].splits * mn : nullptr;
    }
    gx = std::max(gx, P[i].gx);
    gy = std::max(gy, P[i].gy);
    flops += 2.0 * q.M * (q.N_alg > 0 ? q.N_alg : q.N) * (double)(q.K_alg > 0 ? q.K_alg : q.K);
  }
  L.kid = P[0].kid;
  if (g.kind == G_TILED) {  // one block range per problem, a 1-D grid
    long long blk = 0;
    for (int i = 0; i < nl; ++i) {
      B.blk0[i] = (int)blk;
      B.gx[i] = (int)P[i].gx;
      B.gy[i] = (int)P[i].gy;
      B.gz[i] = P[i].splits;
      blk += (long long)P[i].gx * P[i].gy * P[i].splits;
    }
    if (blk > INT_MAX) return fail(c, ZL_ERR_INVALID, "GEMM grid of %lld blocks", blk);
    L.gx = (unsigned)blk;
    L.gy = 1;
    L.gz = 1;
  } else {
    L.gx = gx;
    L.gy = gy;
    L.gz = (unsigned)nl;
  }
  L.threads = (unsigned)g.threads;
  L.flops = flops;
  one = true;
  return ZL_OK;
}

// After a planned launch: split-K partials reduced now, or handed to the
// caller's all-layer reduction (seg_out), which also takes tensors written
// directly.
static zl_status finish_batch(zl_ctx* c, const BatchLaunch& L) {
  for (int i = 0; i < L.nl; ++i) {
    const GemmDesc& q = *L.live[i];
    const zk::GemmArgs& a = L.B.g[i];
    if (q.seg_out) {
      zk::ReduceSeg& r = *q.seg_out;
      r = zk::ReduceSeg{};
      r.part = L.part[i];
      r.rowpart = L.part[i] ? a.rowsumA : nullptr;
      r.out = q.C;
      r.rowout = q.rowsum_out;
      r.mn = (long long)q.M * q.N;
      r.cols = q.N;
      r.ldo = q.ldc;
      r.rows = q.rowsum_out ? q.M : 0;
      r.splits = L.P[i].splits;
      continue;
    }
    if (!L.part[i]) continue;
    zk::SplitReduceArgs r{};
    r.part = L.part[i];
    r.out = q.C;
    r.rowpart = a.rowsumA;
    r.rowout = q.rowsum_out;
    r.guard = q.guard;
    r.mn = (long long)q.M * q.N;
    r.cols = q.N;
    r.ldo = q.ldc;
    r.rows = q.rowsum_out ? q.M : 0;
    r.splits = L.P[i].splits;
    zl_status s = launch_splitk_reduce(c, r);
    if (s) return s;
  }
  return ZL_OK;
}

zl_status run_gemm_batch(zl_ctx* c, const GemmDesc* d, int n) {
  BatchLaunch L;
  bool one = false;
  zl_status s = plan_batch(c, d, n, L, one);
  if (s || L.nl == 0) return s;
  if (!one) {
    s = run_gemm_batch(c, L.live[0], 1);
    return s ? s : run_gemm_batch(c, L.live[1], 1);
  }
  c->pending_flops = L.flops;
  c->pending_shape = {L.live[0]->M, L.live[0]->N, L.live[0]->K, L.P[0].splits};
  s = launch(c, L.kid, L.gx, L.gy, L.gz, L.B, 0, L.threads);
  return s ? s : finish_batch(c, L);
}

zl_status run_gemm_bwd(zl_ctx* c, const GemmDesc* w, int nw, const GemmDesc* d, int nd) {
  if (c->merged_bwd && nd > 0) {
    BatchLaunch W, D;
    bool ow = false, od = false;
    zl_status s = plan_batch(c, w, nw, W, ow);
    if (s) return s;
    if (ow && W.nl > 0 && (s = plan_batch(c, d, nd, D, od))) return s;
    int mk = -1;
    if (ow && od && W.nl > 0 && D.nl > 0 && D.kid == gemm_id("zk_gemm_ak_bn_96x128x32_w24_dg_x")) {
      if (W.kid == gemm_id("zk_gemm_am_bn_128x128x32_w24_x"))
        mk = K_GEMM_BWD_128;
      else if (W.kid == gemm_id("zk_gemm_am_bn_64x128x32_w24_x"))
        mk = K_GEMM_BWD_64;
    }
    if (ow && od && W.nl > 0 && D.nl > 0 && D.kid == gemm_id("zk_gemm_ak_bn_128x128x32_w24_dg_x")) {
      if (W.kid == gemm_id("zk_gemm_am_bn_128x128x32_w24_x"))
        mk = K_GEMM_BWD_128_D128;
      else if (W.kid == gemm_id("zk_gemm_am_bn_64x128x32_w24_x"))
        mk = K_GEMM_BWD_64_D128;
    }
    if (mk >= 0) {
      zk::GemmPair a{};
      a.w = W.B;
      a.d = D.B;
      a.nw = (int)W.gx;  // tiled batches: 1-D grids
      const long long blocks = (long long)W.gx + D.gx;
      c->pending_flops = W.flops + D.flops;
      c->pending_shape = {D.live[0]->M, D.live[0]->N, D.live[0]->K, W.P[0].splits};
      s = launch(c, mk, (unsigned)blocks, 1, 1, a, 0, 512);
      if (!s) s = finish_batch(c, W);
      return s ? s : finish_batch(c, D);
    }
  }
  zl_status s = run_gemm_batch(c, w, nw);
  return s || nd == 0 ? s : run_gemm_batch(c, d, nd);
}

zl_status run_gemm(zl_ctx* c, const GemmDesc& d) { return run_gemm_batch(c, &d, 1); }

zl_status launch_sample(zl_ctx* c, const zk::SampleArgs& a) {
  if (a.A <= 32) return launch(c, K_SAMPLE_G32, (unsigned)cdiv(a.rows, kThreads / 32), 1, 1, a);
  if (a.A <= 64) return launch(c, K_SAMPLE_G64, (unsigned)cdiv(a.rows, kThreads / 64), 1, 1, a);
  return launch(c, K_SAMPLE, (unsigned)cdiv(a.rows, kThreads), 1, 1, a);
}

// Sum the component-major [width x blocks] partials of zk_actor_loss over
// blocks into out[width] (zk_row_sum, fixed order).
zl_status reduce_rows(zl_ctx* c, const float* part, int width, int blocks, float* out) {
  zk::RowSumArgs a{};
  a.out = out;
  a.x = part;
  a.rows = width;
  a.cols = blocks;
  a.ldx = blocks;
  return launch(c, K_ROW_SUM, (unsigned)width, 1, 1, a);
}


// Split lanes for `splits` slices: enough that each thread adds at most 32
// (fewer, longer lanes measured faster than 8 slices per lane for the update's
// 32- and 64-slice weight gradients: 23.6 vs 25.3 us per minibatch).
static int reduce_lanes(int splits) {
  int sl = 1;
  while (sl < 64 && sl * 32 < splits) sl <<= 1;
  return sl;
}

int reduce_all_layout(zk::ReduceSeg* segs, int nseg) {
  int blk = 0;
  for (int i = 0; i < nseg; ++i) {
    zk::ReduceSeg& r = segs[i];
    r.lanes = r.part ? reduce_lanes(r.splits) : 1;
    const int per_block = zk::kReduceAllThreads / r.lanes;
    r.blk0 = blk;
    r.nqb = (int)cdiv(cdiv(r.mn, 4), per_block);
    r.nrb = r.rows > 0 ? (int)cdiv(r.rows, per_block) : 0;
    blk += r.nqb + r.nrb;
  }
  return blk;
}

zl_status launch_reduce_all(zl_ctx* c, const zk::ReduceSeg* segs, int nseg, float* sq_part,
                            const int* guard, const zk::FinalizeArgs* tail) {
  if (nseg < 1 || nseg > zk::kMaxReduceSegs)
    return fail(c, ZL_ERR_INVALID, "reduce_all: %d segments", nseg);
  zk::ReduceAllArgs a{};
  for (int i = 0; i < nseg; ++i) a.seg[i] = segs[i];
  a.nseg = nseg;
  a.sq_part = sq_part;
  a.guard = guard;
  const int blocks = reduce_all_layout(a.seg, nseg);
  a.tail_block = -1;
  if (tail) {  // one more block, after the reduction's, with its slot sq_part[blocks]
    a.tail = *tail;
    a.tail.nsq = blocks;
    a.tail_block = blocks;
  }
  return launch(c, K_REDUCE_ALL, (unsigned)(blocks + (tail ? 1 : 0)), 1, 1, a, 0,
                zk::kReduceAllThreads);
}

static std::string code_object_path() {
  if (const char* e = getenv("ZL_CODE_OBJECT")) return e;
  Dl_info info;
  if (dladdr((void*)&zl_init, &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    size_t slash = p.rfind('/');
    std::string dir = slash == std::string::npos ? "." : p.substr(0, slash);
    return dir + "/zealot_kernels.hsaco";
  }
  return "zealot_kernels.hsaco";
}

// ----------------------------------------------------------------- self-test

// Closed-form inputs of CutileGemm::self_test (src/biped/cutile_gemm.rs:711-716).
static float st_val(int i, int j, int seed, int a, int b, int cst, int p) {
  int h = (i * a + j * b + seed * cst) % p;
  return (float)h / ((float)p / 2.0f) - 1.0f;
}

static zl_status self_test(zl_ctx* c, double* worst_out) {
  struct Case {
    int m, n, k;
    bool lt, rt;
  };
  // (m, n, k, lhs_t, rhs_t) of src/biped/cutile_gemm.rs:699-708.
  const Case cases[] = {{12, 300, 45, false, false}, {45, 300, 256, true, false},
                        {256, 45, 300, false, true}, {64, 96, 4096, false, true},
                        {64, 96, 3072, false, true}, {512, 12288, 51, false, false}};
  double worst = 0.0;
  const double tol = 1e-4;  // fp32 MFMA (the cuTile tf32 bound is 5e-2)
  bool force_fail = getenv("ZL_FORCE_SELF_TEST_FAIL") && strcmp(getenv("ZL_FORCE_SELF_TEST_FAIL"), "1") == 0;
  int ci = 0;
  for (const Case& cs : cases) {
    const int m = cs.m, n = cs.n, k = cs.k;
    std::vector<float> L((size_t)m * k), R((size_t)k * n);
    for (int i = 0; i < m; ++i)
      for (int j = 0; j < k; ++j) L[(size_t)i * k + j] = st_val(i, j, ci, 31, 17, 101, 97);
    for (int i = 0; i < k; ++i)
      for (int j = 0; j < n; ++j) R[(size_t)i * n + j] = st_val(i, j, ci + 7, 31, 17, 101, 97);
    std::vector<double> ref((size_t)m * n, 0.0);
    for (int i = 0; i < m; ++i)
      for (int p = 0; p < k; ++p) {
        double l = L[(size_t)i * k + p];
        const float* rr = &R[(size_t)p * n];
        double* o = &ref[(size_t)i * n];
        for (int j = 0; j < n; ++j) o[j] += l * rr[j];
      }
    std::vector<float> Lb = L, Rb = R;
    if (cs.lt)
      for (int i = 0; i < m; ++i)
        for (int j = 0; j < k; ++j) Lb[(size_t)j * m + i] = L[(size_t)i * k + j];
    if (cs.rt)
      for (int i = 0; i < k; ++i)
        for (int j = 0; j < n; ++j) Rb[(size_t)j * k + i] = R[(size_t)i * n + j];
    float *dl = nullptr, *dr = nullptr, *dout = nullptr;
    ZL_HIP(c, hipMalloc((void**)&dl, Lb.size() * 4));
    ZL_HIP(c, hipMalloc((void**)&dr, Rb.size() * 4));
    ZL_HIP(c, hipMalloc((void**)&dout, (size_t)m * n * 4));
    ZL_HIP(c, hipMemcpy(dl, Lb.data(), Lb.size() * 4, hipMemcpyHostToDevice));
    ZL_HIP(c, hipMemcpy(dr, Rb.data(), Rb.size() * 4, hipMemcpyHostToDevice));
    zl_status s = zl_gemm(c, dout, dl, cs.lt, dr, cs.rt, m, n, k);
    std::vector<float> got((size_t)m * n);
    if (!s) {
      ZL_HIP(c, hipStreamSynchronize(c->stream));
      ZL_HIP(c, hipMemcpy(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost));
    }
    hipFree(dl);
    hipFree(dr);
    hipFree(dout);
    if (s) return s;
    double amax = 1e-6, err = 0.0;
    for (double v : ref) amax = std::max(amax, std::fabs(v));
    for (size_t i = 0; i < ref.size(); ++i) err = std::max(err, std::fabs(got[i] - ref[i]) / amax);
    if (force_fail) err = 1.0;
    if (!(err <= tol))
      return fail(c, ZL_ERR_SELF_TEST, "self-test case %d (m=%d n=%d k=%d lt=%d rt=%d): rel err %.3e",
                  ci, m, n, k, (int)cs.lt, (int)cs.rt, err);
    worst = std::max(worst, err);
    ++ci;
  }
  // Fused bias + ELU with a strided bias column, then the ELU backward and
  // the row sums (src/biped/cutile_gemm.rs:749-826).
  {
    const int m = 100, n = 300, k = 45;
    auto f = [](int i, int j, int seed) { return st_val(i, j, seed, 29, 13, 89, 83); };
    std::vector<float> L((size_t)m * k), R((size_t)k * n), Bb((size_t)m * 8), G((size_t)m * n);
    for (int i = 0; i < m; ++i)
      for (int j = 0; j < k; ++j) L[(size_t)i * k + j] = f(i, j, 1);
    for (int i = 0; i < k; ++i)
      for (int j = 0; j < n; ++j) R[(size_t)i * n + j] = f(i, j, 2);
    for (int i = 0; i < m; ++i)
      for (int j = 0; j < 8; ++j) Bb[(size_t)i * 8 + j] = f(i, j, 3);
    for (int i = 0; i < m; ++i)
      for (int j = 0; j < n; ++j) G[(size_t)i * n + j] = f(i, j, 4);
    std::vector<double> ref((size_t)m * n);
    for (int i = 0; i < m; ++i)
      for (int j = 0; j < n; ++j) {
        double z = 0.0;
        for (int p = 0; p < k; ++p) z += (double)L[(size_t)i * k + p] * R[(size_t)p * n + j];
        z += Bb[(size_t)i * 8];
        ref[(size_t)i * n + j] = z > 0.0 ? z : std::exp(z) - 1.0;
      }
    float *dl, *dr, *db, *dout, *dg, *ds;
    ZL_HIP(c, hipMalloc((void**)&dl, L.size() * 4));
    ZL_HIP(c, hipMalloc((void**)&dr, R.size() * 4));
    ZL_HIP(c, hipMalloc((void**)&db, Bb.size() * 4));
    ZL_HIP(c, hipMalloc((void**)&dout, (size_t)m * n * 4));
    ZL_HIP(c, hipMalloc((void**)&dg, G.size() * 4));
    ZL_HIP(c, hipMalloc((void**)&ds, (size_t)m * 4));
    ZL_HIP(c, hipMemcpy(dl, L.data(), L.size() * 4, hipMemcpyHostToDevice));
    ZL_HIP(c, hipMemcpy(dr, R.data(), R.size() * 4, hipMemcpyHostToDevice));
    ZL_HIP(c, hipMemcpy(db, Bb.data(), Bb.size() * 4, hipMemcpyHostToDevice));
    ZL_HIP(c, hipMemcpy(dg, G.data(), G.size() * 4, hipMemcpyHostToDevice));
    zl_status s = zl_gemm_bias_act(c, dout, dl, dr, m, n, k, db, 8, 1);
    if (!s) s = zl_elu_backward(c, dg, dout, m, n);
    if (!s) s = zl_row_sum(c, ds, dg, m, n);
    std::vector<float> got((size_t)m * n), got_g((size_t)m * n), got_s(m);
    if (!s) {
      ZL_HIP(c, hipStreamSynchronize(c->stream));
      ZL_HIP(c, hipMemcpy(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost));
      ZL_HIP(c, hipMemcpy(got_g.data(), dg, got_g.size() * 4, hipMemcpyDeviceToHost));
      ZL_HIP(c, hipMemcpy(got_s.data(), ds, got_s.size() * 4, hipMemcpyDeviceToHost));
    }
    hipFree(dl);
    hipFree(dr);
    hipFree(db);
    hipFree(dout);
    hipFree(dg);
    hipFree(ds);
    if (s) return s;
    double amax = 1e-6, err = 0.0, err_g = 0.0, err_s = 0.0;
    for (double v : ref) amax = std::max(amax, std::fabs(v));
    for (int i = 0; i < m; ++i) {
      double rs = 0.0;
      for (int j = 0; j < n; ++j) {
        const size_t ix = (size_t)i * n + j;
        const double y = ref[ix];
        err = std::max(err, std::fabs(got[ix] - y) / amax);
        const double gref = G[ix] * (y > 0.0 ? 1.0 : y + 1.0);
        err_g = std::max(err_g, std::fabs(got_g[ix] - gref));
        rs += got_g[ix];
      }
      err_s = std::max(err_s, std::fabs(got_s[i] - rs) / std::max(std::fabs(rs), 1.0));
    }
    if (!(err <= tol && err_g <= tol && err_s <= tol))
      return fail(c, ZL_ERR_SELF_TEST,
                  "self-test fused bias+elu: err %.3e, backward err %.3e, row_sum err %.3e", err,
                  err_g, err_s);
    worst = std::max(worst, std::max(err, std::max(err_g, err_s)));
  }
  *worst_out = worst;
  return ZL_OK;
}

}  // namespace zl

using namespace zl;

extern "C" {

const char* zl_version(void) { return "zealot_hip 0.1.0 (gfx950, fp32 MFMA)"; }

void zl_abi_struct_sizes(size_t out[3]) {
  out[0] = sizeof(zl_ppo_config);
  out[1] = sizeof(zl_batch);
  out[2] = sizeof(zl_ppo_stats);
}

const char* zl_global_error(void) { return g_init_error.c_str(); }

zl_status zl_init(int device, zl_ctx** out) {
  if (!out) return fail(nullptr, ZL_ERR_INVALID, "zl_init: out is NULL");
  *out = nullptr;
  g_init_error.clear();
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0)
    return fail(nullptr, ZL_ERR_HIP, "zl_init: no HIP device (%s)",
                e != hipSuccess ? hipGetErrorString(e) : "count 0");
  if (device < 0 || device >= count)
    return fail(nullptr, ZL_ERR_INVALID, "zl_init: device %d out of range [0, %d)", device, count);
  e = hipSetDevice(device);
  if (e != hipSuccess)
    return fail(nullptr, ZL_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess)
    return fail(nullptr, ZL_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, ZL_ERR_CODE_OBJECT, "zl_init: device is %s, the code object is gfx950",
                prop.gcnArchName);
  zl_ctx* c = new zl_ctx();
  c->device = device;
  c->cu_count = prop.multiProcessorCount;
  std::string path = code_object_path();
  e = hipModuleLoad(&c->module, path.c_str());
  if (e != hipSuccess) {
    fail(nullptr, ZL_ERR_CODE_OBJECT, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
    delete c;
    return ZL_ERR_CODE_OBJECT;
  }
  c->fn.assign(kernel_count(), nullptr);
  for (int k = 0; k < kernel_count(); ++k) {
    e = hipModuleGetFunction(&c->fn[k], c->module, kernel_name(k));
    if (e != hipSuccess) {
      fail(nullptr, ZL_ERR_CODE_OBJECT, "kernel %s not in %s: %s", kernel_name(k), path.c_str(),
           hipGetErrorString(e));
      hipModuleUnload(c->module);
      delete c;
      return ZL_ERR_CODE_OBJECT;
    }
  }
  // Tuning overrides (see zl_ctx).
  const char* lay_env[4] = {"ZL_GEMM_AKBK", "ZL_GEMM_AKBN", "ZL_GEMM_AMBN", "ZL_GEMM_AMBK"};
  for (int l = 0; l < 4; ++l) {
    const char* v = getenv(lay_env[l]);
    if (!v || !*v) continue;
    const int id = gemm_id(v);
    if (id < 0 || layout_of(kGemmTable[id - K_GEMM_BASE].a_kc, kGemmTable[id - K_GEMM_BASE].b_kc) != l) {
      fail(nullptr, ZL_ERR_INVALID, "%s=%s is not a GEMM variant of that layout", lay_env[l], v);
      hipModuleUnload(c->module);
      delete c;
      return ZL_ERR_INVALID;
    }
    c->force_gemm[l] = id;
  }
  if (const char* v = getenv("ZL_SPLITK")) c->force_splits = std::max(0, atoi(v));
  if (const char* v = getenv("ZL_SPLITK_TARGET")) c->splitk_target = std::max(1, atoi(v));
  if (const char* v = getenv("ZL_BWD_SPLIT_DIV")) c->bwd_split_div = std::max(0, atoi(v));
  if (const char* v = getenv("ZL_NARROW")) c->narrow = atoi(v) != 0;
  if (const char* v = getenv("ZL_NARROW_TARGET")) c->narrow_target = std::max(1, atoi(v));
  if (const char* v = getenv("ZL_MERGED_BWD")) c->merged_bwd = atoi(v) != 0;
  if (const char* v = getenv("ZL_POLICY_FUSED")) c->fused_policy = atoi(v) != 0;
  if (const char* v = getenv("ZL_SMALLK")) c->smallk = std::max(0, atoi(v));
  if (const char* v = getenv("ZL_SMALLK_WAVES")) c->smallk_waves = atoi(v) == 8 ? 8 : 4;
  // Default-priority stream (no priority variants are used anywhere).
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    fail(nullptr, ZL_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
    hipModuleUnload(c->module);
    delete c;
    return ZL_ERR_HIP;
  }
  noalloc_setup(c);
  double worst = 0.0;
  zl_status s = self_test(c, &worst);
  if (s) {
    g_init_error = c->err;
    zl_destroy(c);
    return s;
  }
  c->self_test_err = worst;
  c->err.clear();
  *out = c;
  return ZL_OK;
}

zl_status zl_timing_begin(zl_ctx* c, const char* kernel_name) {
  if (!c || !kernel_name) return ZL_ERR_INVALID;
  int id = -1;
  if (strcmp(kernel_name, "*") == 0) {
    id = kTimeAll;
  } else {
    for (int k = 0; k < kernel_count(); ++k)
      if (strcmp(kernel_name, zl::kernel_name(k)) == 0) id = k;
  }
  if (id == -1) return fail(c, ZL_ERR_INVALID, "zl_timing_begin: unknown kernel %s", kernel_name);
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  c->timing_kernel = id;
  c->ev_used = 0;
  return ZL_OK;
}

zl_status zl_timing_end(zl_ctx* c, double* total_ms, long long* launches, double* flops) {
  if (!c) return ZL_ERR_INVALID;
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  const int nk = kernel_count();
  c->rep_ms.assign(nk, 0.0);
  c->rep_flops.assign(nk, 0.0);
  c->rep_launches.assign(nk, 0);
  double tot = 0.0, fl = 0.0;
  c->last_kernel.assign(c->ev_kernel.begin(), c->ev_kernel.begin() + c->ev_used);
  c->last_flops.assign(c->ev_flops.begin(), c->ev_flops.begin() + c->ev_used);
  c->last_shape.assign(c->ev_shape.begin(), c->ev_shape.begin() + c->ev_used);
  c->last_ms.assign(c->ev_used, 0.0);
  for (size_t i = 0; i < c->ev_used; ++i) {
    float ms = 0.f;
    ZL_HIP(c, hipEventElapsedTime(&ms, c->ev_pool[2 * i], c->ev_pool[2 * i + 1]));
    c->last_ms[i] = ms;
    tot += ms;
    fl += c->ev_flops[i];
    const int k = c->ev_kernel[i];
    c->rep_ms[k] += ms;
    c->rep_flops[k] += c->ev_flops[i];
    c->rep_launches[k] += 1;
  }
  if (total_ms) *total_ms = tot;
  if (launches) *launches = (long long)c->ev_used;
  if (flops) *flops = fl;
  c->timing_kernel = -1;
  c->ev_used = 0;
  return ZL_OK;
}

int zl_kernel_count(void) { return kernel_count(); }

zl_status zl_timing_kernel(const zl_ctx* c, int id, const char** name, double* total_ms,
                           long long* launches, double* flops) {
  if (!c || id < 0 || id >= kernel_count()) return ZL_ERR_INVALID;
  if (name) *name = zl::kernel_name(id);
  const bool have = (size_t)id < c->rep_ms.size();
  if (total_ms) *total_ms = have ? c->rep_ms[id] : 0.0;
  if (launches) *launches = have ? c->rep_launches[id] : 0;
  if (flops) *flops = have ? c->rep_flops[id] : 0.0;
  return ZL_OK;
}

long long zl_timing_launch_count(const zl_ctx* c) { return c ? (long long)c->last_ms.size() : 0; }

zl_status zl_timing_launch(const zl_ctx* c, long long i, const char** name, double* ms,
                           double* flops, int* shape4) {
  if (!c || i < 0 || i >= (long long)c->last_ms.size()) return ZL_ERR_INVALID;
  if (name) *name = zl::kernel_name(c->last_kernel[i]);
  if (ms) *ms = c->last_ms[i];
  if (flops) *flops = c->last_flops[i];
  if (shape4)
    for (int j = 0; j < 4; ++j) shape4[j] = c->last_shape[i][j];
  return ZL_OK;
}

void zl_destroy(zl_ctx* c) {
  if (!c) return;
  if (c->stream) hipStreamSynchronize(c->stream);
  noalloc_release(c);
  for (hipEvent_t e : c->ev_pool) hipEventDestroy(e);
  if (c->ws) hipFree(c->ws);
  if (c->stream) hipStreamDestroy(c->stream);
  if (c->module) hipModuleUnload(c->module);
  delete c;
}

const char* zl_last_error(const zl_ctx* c) { return c ? c->err.c_str() : g_init_error.c_str(); }

void* zl_stream(zl_ctx* c) { return c ? (void*)c->stream : nullptr; }

double zl_self_test_error(const zl_ctx* c) { return c ? c->self_test_err : -1.0; }

zl_status zl_synchronize(zl_ctx* c) {
  if (!c) return ZL_ERR_INVALID;
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  return ZL_OK;
}

zl_status zl_alloc(zl_ctx* c, size_t bytes, void** out) {
  if (!c || !out) return ZL_ERR_INVALID;
  *out = nullptr;
  ZL_HIP(c, hipMalloc(out, std::max<size_t>(bytes, 4)));
  return ZL_OK;
}

zl_status zl_free(zl_ctx* c, void* p) {
  if (!c) return ZL_ERR_INVALID;
  if (!p) return ZL_OK;
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  ZL_HIP(c, hipFree(p));
  return ZL_OK;
}

zl_status zl_upload(zl_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return ZL_ERR_INVALID;
  if (!bytes) return ZL_OK;
  ZL_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  return ZL_OK;
}

zl_status zl_download(zl_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return ZL_ERR_INVALID;
  if (!bytes) return ZL_OK;
  ZL_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  return ZL_OK;
}

zl_status zl_copy_d2d(zl_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return ZL_ERR_INVALID;
  if (!bytes) return ZL_OK;
  ZL_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->stream));
  return ZL_OK;
}

// ------------------------------------------------------------- operators

zl_status zl_gemm(zl_ctx* c, float* out, const float* lhs, int lhs_t, const float* rhs, int rhs_t,
                  int m, int n, int k) {
  if (!c) return ZL_ERR_INVALID;
  if (!out || !lhs || !rhs || m < 0 || n < 0 || k < 0)
    return fail(c, ZL_ERR_INVALID, "zl_gemm: bad argument (m=%d n=%d k=%d)", m, n, k);
  GemmDesc d;
  d.A = lhs;
  d.a_kc = !lhs_t;
  d.lda = lhs_t ? m : k;
  d.B = rhs;
  d.b_kc = rhs_t != 0;
  d.ldb = rhs_t ? k : n;
  d.C = out;
  d.ldc = n;
  d.M = m;
  d.N = n;
  d.K = k;
  return run_gemm(c, d);
}

zl_status zl_gemm_bias_act(zl_ctx* c, float* out, const float* lhs, const float* rhs, int m, int n,
                           int k, const float* bias, int bias_row_stride, int elu) {
  if (!c) return ZL_ERR_INVALID;
  if (!out || !lhs || !rhs || !bias || m < 0 || n < 0 || k < 0 || bias_row_stride < 1)
    return fail(c, ZL_ERR_INVALID, "zl_gemm_bias_act: bad argument");
  GemmDesc d;
  d.A = lhs;
  d.a_kc = true;
  d.lda = k;
  d.B = rhs;
  d.b_kc = false;
  d.ldb = n;
  d.C = out;
  d.ldc = n;
  d.M = m;
  d.N = n;
  d.K = k;
  d.epi = zk::kEpiBiasM;
  d.bias = bias;
  d.bias_stride = bias_row_stride;
  d.act = elu ? 1 : 0;
  return run_gemm(c, d);
}

zl_status zl_elu_backward(zl_ctx* c, float* g, const float* y, int m, int n) {
  if (!c) return ZL_ERR_INVALID;
  if (!g || !y || m < 0 || n < 0) return fail(c, ZL_ERR_INVALID, "zl_elu_backward: bad argument");
  zk::EluBwdArgs a{};
  a.g = g;
  a.y = y;
  a.rows = m;
  a.cols = n;
  a.ldg = n;
  a.ldy = n;
  return launch(c, K_ELU_BACKWARD, (unsigned)cdiv((long long)m * n, kThreads), 1, 1, a);
}

zl_status zl_row_sum(zl_ctx* c, float* out, const float* x, int m, int n) {
  if (!c) return ZL_ERR_INVALID;
  if (!out || !x || m < 0 || n < 0) return fail(c, ZL_ERR_INVALID, "zl_row_sum: bad argument");
  zk::RowSumArgs a{};
  a.out = out;
  a.x = x;
  a.rows = m;
  a.cols = n;
  a.ldx = n;
  return launch(c, K_ROW_SUM, (unsigned)m, 1, 1, a);
}

// Sum the [blocks x width] partials over blocks into out[width] (fixed order).
static zl_status reduce_partials(zl_ctx* c, const float* part, int blocks, int width, float* out) {
  zk::SplitReduceArgs r{};
  r.part = part;
  r.out = out;
  r.mn = width;
  r.cols = width;
  r.ldo = width;
  r.splits = blocks;
  return launch_splitk_reduce(c, r);
}

zl_status zl_ppo_actor_grad(zl_ctx* c, const float* mean, int ld_mean, const float* action,
                            int ld_action, const float* log_std, const float* adv,
                            const float* logp_old, const float* mean_old, int ld_mean_old,
                            int rows, int A, float clip, float entropy_coef, float scale,
                            float* d_mean, int ld_d_mean, float* d_log_std, float* stats_dev,
                            int feature_major) {
  if (!c) return ZL_ERR_INVALID;
  // Batch-major rows need ld >= A; feature-major component rows need ld >= rows.
  const int min_ld = feature_major ? rows : A;
  if (!mean || !action || !log_std || !adv || !logp_old || !d_mean || !d_log_std || !stats_dev ||
      rows < 0 || A < 1 || A > 48 || ld_mean < min_ld || ld_action < min_ld || ld_d_mean < min_ld ||
      (mean_old && ld_mean_old < min_ld))
    return fail(c, ZL_ERR_INVALID, "zl_ppo_actor_grad: bad argument (rows=%d A=%d)", rows, A);
  const LossShape sh = actor_loss_shape(rows, A);
  const int nb = sh.blocks;
  const size_t need = (size_t)nb * A + (size_t)nb * 2;
  zl_status s = ensure_ws(c, need);
  if (s) return s;
  zk::ActorLossArgs a{};
  a.mean = mean;
  a.action = action;
  a.adv = adv;
  a.logp_old = logp_old;
  a.mean_old = mean_old;
  a.log_std = log_std;
  a.delta = d_mean;
  a.gls_part = c->ws;
  a.stat_part = c->ws + (size_t)nb * A;
  if (feature_major) {
    a.ldm = a.ldact = a.ldmo = a.ldd = 1;
    a.cm = ld_mean;
    a.cact = ld_action;
    a.cmo = ld_mean_old;
    a.cdd = ld_d_mean;
  } else {
    a.ldm = ld_mean;
    a.ldact = ld_action;
    a.ldmo = ld_mean_old;
    a.ldd = ld_d_mean;
    a.cm = a.cact = a.cmo = a.cdd = 1;
  }
  a.row0 = 0;
  a.rows = rows;
  a.A = A;
  a.clip = clip;
  a.entropy_coef = entropy_coef;
  a.scale = scale;
  a.rows_per_block = sh.rows_per_block;
  a.group = sh.group;
  if (nb == 0) return ZL_OK;
  s = launch(c, sh.kernel, (unsigned)nb, 1, 1, a, 0, zk::kLossThreads);
  if (s) return s;
  s = reduce_rows(c, a.gls_part, A, nb, d_log_std);
  if (s) return s;
  return reduce_rows(c, a.stat_part, 2, nb, stats_dev);
}

zl_status zl_ppo_value_grad(zl_ctx* c, const float* v, const float* value_old, const float* ret,
                            int rows, float clip, float value_coef, float scale, float* d_v,
                            float* stats_dev) {
  if (!c) return ZL_ERR_INVALID;
  if (!v || !value_old || !ret || !d_v || !stats_dev || rows < 0)
    return fail(c, ZL_ERR_INVALID, "zl_ppo_value_grad: bad argument");
  const int nb = (int)cdiv(rows, kThreads);
  if (nb == 0) return ZL_OK;
  zl_status s = ensure_ws(c, (size_t)nb);
  if (s) return s;
  zk::ValueLossArgs a{};
  a.v = v;
  a.value_old = value_old;
  a.ret = ret;
  a.delta = d_v;
  a.stat_part = c->ws;
  a.ldv = 1;
  a.ldd = 1;
  a.rows = rows;
  a.clip = clip;
  a.value_coef = value_coef;
  a.scale = scale;
  s = launch(c, K_VALUE_LOSS, (unsigned)nb, 1, 1, a);
  if (s) return s;
  return reduce_partials(c, c->ws, nb, 1, stats_dev);
}

zl_status zl_adam_step(zl_ctx* c, float* p, const float* g, float* m, float* v, size_t n, float lr,
                       float beta1, float beta2, float eps, float bc1, float bc2) {
  if (!c) return ZL_ERR_INVALID;
  if (!p || !g || !m || !v) return fail(c, ZL_ERR_INVALID, "zl_adam_step: null pointer");
  zk::AdamArgs a{};
  a.p = p;
  a.g = g;
  a.m = m;
  a.v = v;
  a.n = (long long)n;
  a.end_a = (long long)n;
  a.end_c = (long long)n;
  a.lr = lr;
  a.bc1 = bc1;
  a.bc2 = bc2;
  a.beta1 = beta1;
  a.beta2 = beta2;
  a.eps = eps;
  return launch(c, K_ADAM, (unsigned)cdiv((long long)n, 4 * kThreads), 1, 1, a);
}

zl_status zl_grad_sqnorm(zl_ctx* c, const float* x, size_t n, float* out_dev) {
  if (!c) return ZL_ERR_INVALID;
  if (!x || !out_dev) return fail(c, ZL_ERR_INVALID, "zl_grad_sqnorm: null pointer");
  const int chunk = 2048;
  const int nb = std::max(1, (int)cdiv((long long)n, chunk));
  zl_status s = ensure_ws(c, (size_t)nb);
  if (s) return s;
  zk::SumsqArgs a{};
  a.x = x;
  a.part = c->ws;
  a.off0 = 0;
  a.len0 = (long long)n;
  a.blocks0 = nb;
  a.chunk = chunk;
  s = launch(c, K_SUMSQ, (unsigned)nb, 1, 1, a);
  if (s) return s;
  return reduce_partials(c, c->ws, nb, 1, out_dev);
}

zl_status zl_grad_clip_scale(zl_ctx* c, const zl_tensor* tensors, int count, float max_norm,
                             float* scale_dev, float* norm_dev) {
  if (!c) return ZL_ERR_INVALID;
  if (!tensors || !scale_dev || count < 1 || count > zk::kMaxNormTensors)
    return fail(c, ZL_ERR_INVALID, "zl_grad_clip_scale: bad argument (count %d)", count);
  zk::SumsqMultiArgs a{};
  const int chunk = 2048;
  int blk = 0;
  for (int j = 0; j < count; ++j) {
    if (!tensors[j].ptr && tensors[j].n)
      return fail(c, ZL_ERR_INVALID, "zl_grad_clip_scale: tensor %d is NULL", j);
    a.x[j] = tensors[j].ptr;
    a.n[j] = (long long)tensors[j].n;
    a.blk0[j] = blk;
    blk += (int)std::max<long long>(1, cdiv((long long)tensors[j].n, chunk));
  }
  a.blk0[count] = blk;
  a.count = count;
  a.chunk = chunk;
  zl_status s = ensure_ws(c, (size_t)blk);
  if (s) return s;
  a.part = c->ws;
  if ((s = launch(c, K_SUMSQ_MULTI, (unsigned)blk, 1, 1, a))) return s;
  zk::ClipScaleArgs cs{};
  cs.part = c->ws;
  cs.nparts = blk;
  cs.max_norm = max_norm;
  cs.scale = scale_dev;
  cs.norm = norm_dev;
  return launch(c, K_CLIP_SCALE, 1, 1, 1, cs, 0, 64);
}

// zl_adam_multi (part == nullptr) or its clipped form (the scale taken in
// every block from `nparts` sum-of-squares partials at `part`).
static zl_status adam_multi_launch(zl_ctx* c, const zl_adam_tensor* tensors, int count, float lr,
                                   float beta1, float beta2, float eps, float bc1, float bc2,
                                   const float* clip_scale_dev, const float* part, int nparts,
                                   float max_norm, float* scale_out, float* norm_out) {
  zk::AdamMultiArgs a{};
  a.part = part;
  a.nparts = nparts;
  a.max_norm = max_norm;
  a.scale_out = scale_out;
  a.norm_out = norm_out;
  int blk = 0;
  for (int j = 0; j < count; ++j) {
    const zl_adam_tensor& t = tensors[j];
    if (t.n && (!t.p || !t.g || !t.m || !t.v))
      return fail(c, ZL_ERR_INVALID, "zl_adam_multi: tensor %d has a NULL pointer", j);
    a.t[j].p = t.p;
    a.t[j].g = t.g;
    a.t[j].m = t.m;
    a.t[j].v = t.v;
    a.t[j].n = (long long)t.n;
    a.blk0[j] = blk;
    blk += (int)cdiv((long long)t.n, 4 * kThreads);
  }
  a.blk0[count] = blk;
  a.count = count;
  a.scale = clip_scale_dev;
  a.lr = lr;
  a.bc1 = bc1;
  a.bc2 = bc2;
  a.beta1 = beta1;
  a.beta2 = beta2;
  a.eps = eps;
  return launch(c, K_ADAM_MULTI, (unsigned)blk, 1, 1, a);
}

zl_status zl_adam_multi(zl_ctx* c, const zl_adam_tensor* tensors, int count, float lr, float beta1,
                        float beta2, float eps, float bc1, float bc2, const float* clip_scale_dev) {
  if (!c) return ZL_ERR_INVALID;
  if (!tensors || count < 1 || count > zk::kMaxAdamTensors)
    return fail(c, ZL_ERR_INVALID, "zl_adam_multi: bad argument (count %d)", count);
  return adam_multi_launch(c, tensors, count, lr, beta1, beta2, eps, bc1, bc2, clip_scale_dev,
                           nullptr, 0, 0.0f, nullptr, nullptr);
}

zl_status zl_adam_multi_clip(zl_ctx* c, const zl_adam_tensor* tensors, int count, float lr,
                             float beta1, float beta2, float eps, float bc1, float bc2,
                             float max_norm, float* scale_dev, float* norm_dev) {
  if (!c) return ZL_ERR_INVALID;
  if (!tensors || count < 1 || count > zk::kMaxAdamTensors || count > zk::kMaxNormTensors)
    return fail(c, ZL_ERR_INVALID, "zl_adam_multi_clip: bad argument (count %d)", count);
  // The partials of zl_grad_clip_scale over the gradients, same chunking.
  zk::SumsqMultiArgs q{};
  const int chunk = 2048;
  int blk = 0;
  for (int j = 0; j < count; ++j) {
    const zl_adam_tensor& t = tensors[j];
    if (t.n && (!t.p || !t.g || !t.m || !t.v))
      return fail(c, ZL_ERR_INVALID, "zl_adam_multi_clip: tensor %d has a NULL pointer", j);
    q.x[j] = t.g;
    q.n[j] = (long long)t.n;
    q.blk0[j] = blk;
    blk += (int)std::max<long long>(1, cdiv((long long)t.n, chunk));
  }
  q.blk0[count] = blk;
  q.count = count;
  q.chunk = chunk;
  zl_status s = ensure_ws(c, (size_t)blk);
  if (s) return s;
  q.part = c->ws;
  if ((s = launch(c, K_SUMSQ_MULTI, (unsigned)blk, 1, 1, q))) return s;
  return adam_multi_launch(c, tensors, count, lr, beta1, beta2, eps, bc1, bc2, nullptr, c->ws, blk,
                           max_norm, scale_dev, norm_dev);
}

zl_status zl_gae(zl_ctx* c, const float* rewards, const float* values, const uint8_t* dones,
                 const float* last_values, int T, int N, long long in_ts, long long in_es,
                 long long out_ts, long long out_es, float gamma, float lam, float* adv,
                 float* ret) {
  if (!c) return ZL_ERR_INVALID;
  if (!rewards || !values || !dones || !last_values || !adv || !ret || T < 0 || N < 0)
    return fail(c, ZL_ERR_INVALID, "zl_gae: bad argument");
  if (T == 0 || N == 0) return ZL_OK;  // no steps or no envs: nothing to write
  zk::GaeArgs a{};
  a.r = rewards;
  a.v = values;
  a.done = dones;
  a.last_v = last_values;
  a.adv = adv;
  a.ret = ret;
  a.in_ts = in_ts;
  a.in_es = in_es;
  a.out_ts = out_ts;
  a.out_es = out_es;
  a.T = T;
  a.N = N;
  a.gamma = gamma;
  a.lam = lam;
  return launch(c, K_GAE, (unsigned)cdiv(N, zk::kGaeThreads), 1, 1, a, 0, zk::kGaeThreads);
}

}  // extern "C"

namespace zl {
// Three-launch deterministic normalisation with caller scratch (2*nparts
// floats); the last phase also writes the result to *wb when wb is set.
zl_status adv_normalize_into(zl_ctx* c, float* adv, long long n, float* scratch, int nparts,
                             int chunk, const int* guard, float* const* wb) {
  zk::AdvNormArgs a{};
  a.wb = wb;
  a.x = adv;
  a.part = scratch;
  a.part2 = scratch + nparts;
  a.guard = guard;
  a.n = n;
  a.nparts = nparts;
  a.chunk = chunk;
  for (int ph = 0; ph < 3; ++ph) {
    a.phase = ph;
    zl_status s = launch(c, K_ADV_NORM, (unsigned)nparts, 1, 1, a);
    if (s) return s;
  }
  return ZL_OK;
}
}  // namespace zl

extern "C" {

zl_status zl_adv_normalize(zl_ctx* c, float* adv, size_t n) {
  if (!c) return ZL_ERR_INVALID;
  if (!adv || n == 0) return fail(c, ZL_ERR_INVALID, "zl_adv_normalize: bad argument");
  const int chunk = 4096;
  const int nparts = (int)cdiv((long long)n, chunk);
  zl_status s = ensure_ws(c, (size_t)2 * nparts);
  if (s) return s;
  return adv_normalize_into(c, adv, (long long)n, c->ws, nparts, chunk, nullptr, nullptr);
}

zl_status zl_sample_actions(zl_ctx* c, const float* mean, int ld_mean, const float* log_std,
                            const float* eps, int rows, int A, float* action, float* logp) {
  if (!c) return ZL_ERR_INVALID;
  if (!mean || !log_std || !eps || !action || !logp || rows < 0 || A < 1 || ld_mean < A)
    return fail(c, ZL_ERR_INVALID, "zl_sample_actions: bad argument");
  zk::SampleArgs a{};
  a.mean = mean;
  a.log_std = log_std;
  a.eps = eps;
  a.action = action;
  a.logp = logp;
  a.rows = rows;
  a.A = A;
  a.ldm = ld_mean;
  a.lde = A;
  a.lda = A;
  return launch_sample(c, a);
}

}  // extern "C"
