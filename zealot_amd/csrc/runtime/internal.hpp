// internal.hpp — host-side internals of libzealot_hip.so.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <array>
#include <string>
#include <vector>

#include "../kernels/zk_args.h"
#include "zealot_hip.h"

namespace zl {

// Kernels of the code object. The fixed kernels come first; the GEMM
// variants (one per layout / tile / wave grid) follow from K_GEMM_BASE.
enum KernelId : int {
  K_SPLITK_REDUCE = 0,
  K_ACTOR_LOSS,
  K_VALUE_LOSS,
  K_SUMSQ,
  K_ADAM,
  K_EPOCH_BEGIN,
  K_KL,
  K_EPOCH_END,
  K_GAE,
  K_ADV_NORM,
  K_ELU_BACKWARD,
  K_ROW_SUM,
  K_COPY_ROWS,
  K_SAMPLE,
  K_CLAMP,
  K_REDUCE_ALL,
  K_ACTOR_LOSS_G64,
  K_HEAD,
  K_NORM_SET,
  K_NORM_APPLY,
  K_NORM_STATS,
  K_NORM_MERGE,
  K_NORM_COMMIT,
  K_SAMPLE_G32,
  K_SAMPLE_G64,
  K_STAGE,
  K_SUMSQ_MULTI,
  K_CLIP_SCALE,
  K_ADAM_MULTI,
  K_GEMM_BWD_128,
  K_GEMM_BWD_64,
  K_GEMM_BWD_128_D128,
  K_GEMM_BWD_64_D128,
  K_HEAD_FWD,
  K_HEAD_FWD_X,
  K_POLICY,
  K_TRANSPOSE,
  K_POLICY_PACK,
  K_GEMM_BASE
};

// Kernel family of a GEMM variant: LDS-tiled (gemm_mfma.hip) or one of the
// register-resident narrow kernels (narrow.hip): N <= 32 (forward of an
// output layer), K <= 32 (its data gradient), M <= 32 (its weight gradient).
enum GemmKind : int { G_TILED = 0, G_NARROW_N = 1, G_NARROW_K = 2, G_NARROW_M = 3 };

// One GEMM variant: operand orientation, tile (for the narrow kernels: rows
// per block and the largest narrow dimension), k-tile, block size, whether it
// loads both operands as float4 rows (vec) or element by element, and family.
struct GemmKernel {
  const char* name;
  bool a_kc, b_kc;
  int bm, bn, bk, threads;
  bool vec;
  int kind = G_TILED;
  bool need_vec_b = false;  // reads B as float4 rows even when A is read by elements
};

// Narrow kernels: 16-row strips, four wavefronts per block; the data-gradient
// form takes 32 columns per block, the weight-gradient form 64 columns and
// row slices in multiples of 4 wavefronts x 16 rows.
constexpr int kNarrowRows = 64;
constexpr int kNarrowKCols = 32;
constexpr int kNarrowCols = 64;
constexpr int kNarrowSliceQuantum = 64;

extern const char* const kFixedNames[K_GEMM_BASE];
extern const GemmKernel kGemmTable[];
extern const int kGemmCount;
int kernel_count();
const char* kernel_name(int id);

constexpr int kThreads = 256;

inline long long round_up(long long x, long long m) { return (x + m - 1) / m * m; }
inline long long cdiv(long long a, long long b) { return (a + b - 1) / b; }

// Launch shape of zk_actor_loss: one lane group (32 lanes for A <= 32, else
// 64) per sample, kLossThreads / group samples in flight per block, and at most
// kLossMaxBlocks blocks over the rows (one partial row each).
constexpr int kLossMaxBlocks = 256;
struct LossShape {
  int group, rows_per_block, blocks;
  int kernel;  // K_ACTOR_LOSS (32-lane groups) or K_ACTOR_LOSS_G64
};
inline LossShape actor_loss_shape(int rows, int A) {
  LossShape s;
  s.group = A <= 32 ? 32 : 64;
  s.kernel = s.group == 32 ? K_ACTOR_LOSS : K_ACTOR_LOSS_G64;
  const int ng = zk::kLossThreads / s.group;
  s.rows_per_block = (int)std::max<long long>(ng, cdiv(rows, kLossMaxBlocks));
  s.blocks = rows > 0 ? (int)cdiv(rows, s.rows_per_block) : 0;
  return s;
}

// GEMM layouts (A K-/M-contiguous x B K-/N-contiguous).
enum GemmLayout : int { L_AK_BK = 0, L_AK_BN = 1, L_AM_BN = 2, L_AM_BK = 3 };
inline int layout_of(bool a_kc, bool b_kc) {
  return a_kc ? (b_kc ? L_AK_BK : L_AK_BN) : (b_kc ? L_AM_BK : L_AM_BN);
}

}  // namespace zl

struct zl_ctx {
  int device = 0;
  int cu_count = 256;  // compute units of the device (zl_init)
  hipStream_t stream = nullptr;
  hipModule_t module = nullptr;
  std::vector<hipFunction_t> fn;  // by kernel id
  std::string err;
  double self_test_err = 0.0;
  // Scratch owned by the context for the stand-alone operators (split-K
  // partials, reduction partials). Grown with a stream sync, never inside a
  // captured graph: composite objects own their scratch.
  float* ws = nullptr;
  size_t ws_floats = 0;
  // Per-launch hipEvent timing of one kernel (zl_timing_begin / _end). While
  // set, composite entry points launch eagerly instead of replaying graphs.
  int timing_kernel = -1;           // kernel id, kTimeAll, or -1 (off)
  std::vector<hipEvent_t> ev_pool;  // pairs: [2i] start, [2i+1] stop
  size_t ev_used = 0;
  std::vector<int> ev_kernel;       // kernel id of timed launch i
  std::vector<double> ev_flops;     // algorithmic FLOP of timed launch i
  std::vector<std::array<int, 4>> ev_shape;  // GEMM M, N, K, splits of timed launch i
  double pending_flops = 0.0;       // set by run_gemm for the next launch
  std::array<int, 4> pending_shape{};  // likewise
  // Per-kernel results of the last finished timing session, and its
  // launches in issue order (kernel id, ms, FLOP, GEMM shape).
  std::vector<double> rep_ms, rep_flops;
  std::vector<long long> rep_launches;
  std::vector<int> last_kernel;
  std::vector<double> last_ms, last_flops;
  std::vector<std::array<int, 4>> last_shape;
  // Tuning overrides (environment, read at zl_init): forced GEMM variant per
  // layout (ZL_GEMM_AKBK / _AKBN / _AMBN / _AMBK), split-K slice count
  // (ZL_SPLITK) and the split-K target grid size (ZL_SPLITK_TARGET).
  int force_gemm[4] = {-1, -1, -1, -1};
  int force_splits = 0;
  int splitk_target = 256;
  // Divisor of the split-K slice count of weight gradients that share a
  // launch with their layer's data gradients (ZL_BWD_SPLIT_DIV; 0: the
  // rule in pair_backward).
  int bwd_split_div = 0;
  // Narrow kernels for shapes with a dimension <= 32 (ZL_NARROW=0 turns them
  // off) and the block count their row slices aim at (ZL_NARROW_TARGET).
  bool narrow = true;
  int narrow_target = 256;
  // A layer's weight- and data-gradient GEMMs as one launch where a merged
  // kernel covers their variants (ZL_MERGED_BWD=0 runs them as two).
  bool merged_bwd = true;
  // Forwards of up to kPolicyFusedRows rows (a rollout step) as one zk_policy
  // launch where the nets fit it (ZL_POLICY_FUSED=0 keeps the layer GEMMs).
  bool fused_policy = true;
  // A K-contiguous x B N-contiguous products with K <= 128 and a plain or
  // bias epilogue on the small-K variants (ZL_SMALLK: 0 off, 1 when A rows
  // are not float4-aligned (default), 2 always).
  int smallk = 1;
  int smallk_waves = 8;  // wavefronts per small-K block (ZL_SMALLK_WAVES: 4 or 8; 8 measured 12.8 vs 13.3 us)
  // Device address of the allocation-free scratch array on this context's
  // device (zl_grad_clip_scale_noalloc), set at zl_init.
  float* noalloc_scratch = nullptr;  // this context's slot of the array
  int noalloc_slot = -1;
  hipError_t noalloc_err = hipSuccess;
};

namespace zl {

zl_status fail(zl_ctx* c, zl_status s, const char* fmt, ...);

#define ZL_HIP(c, call)                                                                  \
  do {                                                                                   \
    hipError_t e_ = (call);                                                              \
    if (e_ != hipSuccess)                                                                \
      return ::zl::fail((c), ZL_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
  } while (0)

constexpr int kTimeAll = -2;
zl_status timing_mark(zl_ctx* c, bool stop, int kernel = 0, double flops = 0.0);

template <class Args>
zl_status launch(zl_ctx* c, int k, unsigned gx, unsigned gy, unsigned gz, const Args& a,
                 unsigned shmem = 0, unsigned threads = kThreads) {
  if (gx == 0 || gy == 0 || gz == 0) return ZL_OK;
  const bool timed = c->timing_kernel == k || c->timing_kernel == kTimeAll;
  if (timed) {
    zl_status s = timing_mark(c, false, k, c->pending_flops);
    if (s) return s;
  }
  c->pending_flops = 0.0;
  c->pending_shape = {0, 0, 0, 0};
  void* params[] = {(void*)&a};
  hipError_t e = hipModuleLaunchKernel(c->fn[k], gx, gy, gz, threads, 1, 1, shmem, c->stream,
                                       params, nullptr);
  if (e != hipSuccess)
    return fail(c, ZL_ERR_HIP, "launch %s failed: %s", kernel_name(k), hipGetErrorString(e));
  return timed ? timing_mark(c, true) : ZL_OK;
}

// One GEMM with its epilogue and (optionally) split-K + the fixed-order
// reduction. A/B orientation: a_kc = A K-contiguous ([M][K] storage), else
// M-contiguous ([K][M]); b_kc = B K-contiguous ([N][K]), else N-contiguous
// ([K][N]). perm* remap the storage row index.
struct GemmDesc {
  const float* A = nullptr;
  int lda = 0;
  bool a_kc = true;
  const int* permA = nullptr;
  const float* B = nullptr;
  int ldb = 0;
  bool b_kc = true;
  const int* permB = nullptr;
  float* C = nullptr;
  int ldc = 0;
  int M = 0, N = 0, K = 0;
  // > 0: the N / K of the product itself when N / K run over zero padding
  // (the launch's FLOP count for timing uses these).
  int N_alg = 0, K_alg = 0;
  int epi = zk::kEpiStore;
  const float* bias = nullptr;
  int bias_stride = 1;
  int act = 0;
  const float* Y = nullptr;
  int ldy = 0;
  float* rowsum_out = nullptr;  // row sums of A (bias gradient of a wgrad)
  int splits = 0;               // 0: heuristic; only kEpiStore may split
  const int* guard = nullptr;
  float* ws = nullptr;          // split-K scratch (floats); nullptr: context scratch
  size_t ws_floats = 0;
  zk::ReduceSeg* seg_out = nullptr;  // set: no reduce launch, describe it here instead
};

// Variant choice and split-K decision shared by run_gemm and the scratch
// sizing of composites.
// vec: both operands can be read as aligned float4 rows (see run_gemm).
// vec_b: B alone can be read as float4 rows and the problem has no split-K,
// row sums or gathers (the small-K variants may then take it).
int pick_gemm(const zl_ctx* c, int M, int N, int K, bool a_kc, bool b_kc, bool vec = true,
              int epi = zk::kEpiStore, bool vec_b = false);
int gemm_splits(const zl_ctx* c, int M, int N, int K, bool a_kc, bool b_kc, int epi,
                bool vec = true);
size_t gemm_ws_floats(const zl_ctx* c, int M, int N, int K, bool a_kc, bool b_kc, int epi);
zl_status run_gemm(zl_ctx* c, const GemmDesc& d);
// One launch for n (1 or 2) problems that pick the same variant (else n
// launches); problems that split K over slices need caller scratch when n > 1.
zl_status run_gemm_batch(zl_ctx* c, const GemmDesc* d, int n);
// A layer's backward: the weight-gradient batch w and the data-gradient
// batch d (nd may be 0), as one zk_gemm_bwd_* launch when both are single
// exact-fit launches of the variants it covers, else as run_gemm_batch(w)
// then run_gemm_batch(d).
zl_status run_gemm_bwd(zl_ctx* c, const GemmDesc* w, int nw, const GemmDesc* d, int nd);
// Block layout of zk_reduce_all over `segs` (fills lanes / blk0 / nqb / nrb);
// returns the block count (= number of sum-of-squares partials).
int reduce_all_layout(zk::ReduceSeg* segs, int nseg);
// With `tail`, one extra block runs the minibatch tail (its nsq is set to the
// reduction's block count, the slot of the log_std squared norm in sq_part).
zl_status launch_reduce_all(zl_ctx* c, const zk::ReduceSeg* segs, int nseg, float* sq_part,
                            const int* guard, const zk::FinalizeArgs* tail = nullptr);
// Fixed-order sum over the split slices (zk_splitk_reduce); picks the split
// lanes and grid from the shape. `r.lanes` is set here.
zl_status launch_splitk_reduce(zl_ctx* c, zk::SplitReduceArgs& r);
zl_status ensure_ws(zl_ctx* c, size_t floats);
// out[k] = sum over b of part[k * blocks + b], k < width (zk_row_sum).
zl_status reduce_rows(zl_ctx* c, const float* part, int width, int blocks, float* out);
// Sampling + logp (zk_sample_g32 / _g64 for A <= 32 / 64, else zk_sample).
zl_status launch_sample(zl_ctx* c, const zk::SampleArgs& a);

// Looks up the allocation-free scratch array's address on the context's
// device (defined in noalloc.hip; the device must be current).
void noalloc_setup(zl_ctx* c);
// Gives the context's slot of that array back (zl_destroy).
void noalloc_release(zl_ctx* c);

// zl_ppo internals for the checkpoint code (defined in mlp_ppo.cpp).
zl_ctx* ppo_ctx(zl_ppo* p);
void ppo_dims(const zl_ppo* p, std::vector<int>* actor, std::vector<int>* critic);
// Packed moments (layout of zl_ppo_get_moments), all six non-NULL.
zl_status ppo_set_moments(zl_ppo* p, const float* ma, const float* va, const float* mc,
                          const float* vc, const float* mls, const float* vls);
void ppo_set_counters(zl_ppo* p, int t, unsigned long long gstep);

}  // namespace zl
