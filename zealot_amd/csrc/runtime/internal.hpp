// internal.hpp — host-side internals of libzealot_hip.so.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <string>
#include <vector>

#include "../kernels/zk_args.h"
#include "zealot_hip.h"

namespace zl {

enum KernelId : int {
  K_GEMM_AK_BK_64x128 = 0,
  K_GEMM_AK_BK_128x32,
  K_GEMM_AK_BK_256x16,
  K_GEMM_AK_BN_64x128,
  K_GEMM_AM_BN_64x128,
  K_GEMM_AM_BK_64x128,
  K_SPLITK_REDUCE,
  K_ACTOR_LOSS,
  K_VALUE_LOSS,
  K_SUMSQ,
  K_FINALIZE,
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
  K_COUNT
};

extern const char* const kKernelNames[K_COUNT];

constexpr int kThreads = 256;

inline long long round_up(long long x, long long m) { return (x + m - 1) / m * m; }
inline long long cdiv(long long a, long long b) { return (a + b - 1) / b; }

}  // namespace zl

struct zl_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipModule_t module = nullptr;
  hipFunction_t fn[zl::K_COUNT] = {};
  std::string err;
  double self_test_err = 0.0;
  // Scratch owned by the context for the stand-alone operators (split-K
  // partials, reduction partials). Grown with a stream sync, never inside a
  // captured graph: composite objects own their scratch.
  float* ws = nullptr;
  size_t ws_floats = 0;
  // Per-launch hipEvent timing of one kernel (zl_timing_begin / _end). While
  // set, composite entry points launch eagerly instead of replaying graphs.
  int timing_kernel = -1;
  std::vector<hipEvent_t> ev_pool;  // pairs: [2i] start, [2i+1] stop
  size_t ev_used = 0;
};

namespace zl {

zl_status fail(zl_ctx* c, zl_status s, const char* fmt, ...);

#define ZL_HIP(c, call)                                                                  \
  do {                                                                                   \
    hipError_t e_ = (call);                                                              \
    if (e_ != hipSuccess)                                                                \
      return ::zl::fail((c), ZL_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
  } while (0)

zl_status timing_mark(zl_ctx* c, bool stop);

template <class Args>
zl_status launch(zl_ctx* c, KernelId k, unsigned gx, unsigned gy, unsigned gz, const Args& a,
                 unsigned shmem = 0) {
  if (gx == 0 || gy == 0 || gz == 0) return ZL_OK;
  const bool timed = c->timing_kernel == (int)k;
  if (timed) {
    zl_status s = timing_mark(c, false);
    if (s) return s;
  }
  void* params[] = {(void*)&a};
  hipError_t e = hipModuleLaunchKernel(c->fn[k], gx, gy, gz, kThreads, 1, 1, shmem, c->stream,
                                       params, nullptr);
  if (e != hipSuccess)
    return fail(c, ZL_ERR_HIP, "launch %s failed: %s", kKernelNames[k], hipGetErrorString(e));
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
};

// Split-K decision shared by run_gemm and the scratch sizing of composites.
int gemm_splits(int M, int N, int K, bool a_kc, bool b_kc, int epi);
size_t gemm_ws_floats(int M, int N, int K, bool a_kc, bool b_kc, int epi);
zl_status run_gemm(zl_ctx* c, const GemmDesc& d);
zl_status ensure_ws(zl_ctx* c, size_t floats);

}  // namespace zl
