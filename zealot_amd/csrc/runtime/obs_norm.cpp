// obs_norm.cpp — C-ABI entry points of the device observation normaliser
// (Normalizer / PendingNorm, zealot-rl/src/ppo.rs:104-206); kernels in
// kernels/obs_norm.hip.
#include "internal.hpp"

using namespace zl;

namespace {

zl_status check_dim(zl_ctx* c, const char* fn, int dim) {
  if (dim < 1 || dim > zk::kNormMaxDim)
    return fail(c, ZL_ERR_INVALID, "%s: dim %d outside [1, %d]", fn, dim, zk::kNormMaxDim);
  return ZL_OK;
}

}  // namespace

extern "C" {

zl_status zl_norm_reset(zl_ctx* c, float* state, int dim, int unit_prior) {
  if (!c) return ZL_ERR_INVALID;
  if (zl_status s = check_dim(c, "zl_norm_reset", dim)) return s;
  if (!state) return fail(c, ZL_ERR_INVALID, "zl_norm_reset: null state");
  zk::NormArgs a{};
  a.state = state;
  a.dim = dim;
  a.unit_prior = unit_prior != 0;
  return launch(c, K_NORM_SET, (unsigned)cdiv(2 * dim + 1, kThreads), 1, 1, a);
}

zl_status zl_norm_update(zl_ctx* c, float* state, int dim, const float* x, int ld,
                         long long rows) {
  if (!c) return ZL_ERR_INVALID;
  if (zl_status s = check_dim(c, "zl_norm_update", dim)) return s;
  if (!state || (rows > 0 && !x) || ld < dim || rows < 0)
    return fail(c, ZL_ERR_INVALID, "zl_norm_update: bad argument");
  if (rows == 0) return ZL_OK;
  const long long nchunks = cdiv(rows, zk::kNormChunkRows);
  if (nchunks > INT32_MAX / 2) return fail(c, ZL_ERR_INVALID, "zl_norm_update: too many rows");
  zl_status s = ensure_ws(c, (size_t)nchunks * 2 * dim);
  if (s) return s;
  zk::NormArgs a{};
  a.x = x;
  a.state = state;
  a.part = c->ws;
  a.rows = rows;
  a.dim = dim;
  a.ldx = ld;
  a.nchunks = (int)nchunks;
  if ((s = launch(c, K_NORM_STATS, (unsigned)nchunks, (unsigned)cdiv(dim, 64), 1, a))) return s;
  return launch(c, K_NORM_MERGE, 1, 1, 1, a, 0, zk::kNormFoldThreads);
}

zl_status zl_norm_commit(zl_ctx* c, float* state, float* pending, int dim) {
  if (!c) return ZL_ERR_INVALID;
  if (zl_status s = check_dim(c, "zl_norm_commit", dim)) return s;
  if (!state || !pending || state == pending)
    return fail(c, ZL_ERR_INVALID, "zl_norm_commit: bad argument");
  zk::NormArgs a{};
  a.state = state;
  a.pending = pending;
  a.dim = dim;
  return launch(c, K_NORM_COMMIT, 1, 1, 1, a, 0, zk::kNormFoldThreads);
}

zl_status zl_norm_normalize(zl_ctx* c, const float* state, int dim, const float* x, int ld_x,
                            long long rows, float* out, int ld_out) {
  if (!c) return ZL_ERR_INVALID;
  if (zl_status s = check_dim(c, "zl_norm_normalize", dim)) return s;
  if (!state || rows < 0 || (rows > 0 && (!x || !out)) || ld_x < dim || ld_out < dim ||
      (x == out && ld_x != ld_out))
    return fail(c, ZL_ERR_INVALID, "zl_norm_normalize: bad argument");
  if (rows == 0) return ZL_OK;
  zk::NormArgs a{};
  a.x = x;
  a.out = out;
  a.state = const_cast<float*>(state);
  a.rows = rows;
  a.dim = dim;
  a.ldx = ld_x;
  a.ldo = ld_out;
  // One batch of 4 loads per thread for dim <= 256 (4 passes of 256 / dim
  // rows), 8 rows per block otherwise: thousands of blocks for a rollout
  // batch, enough to fill the chip for one env step. Batches that still give
  // >= 2048 blocks take four such batches per block, which spreads each
  // block's normaliser-state prologue over more rows (the update batch
  // [98,304 x 123]: 23.3 -> 18.6 us by events; eight batches: 20.5).
  const int batch_rows = 4 * (kThreads / dim);
  a.rows_per_block = dim <= kThreads ? (rows >= 8LL * batch_rows * 1024 ? 4 * batch_rows : batch_rows) : 8;
  return launch(c, K_NORM_APPLY, (unsigned)cdiv(rows, a.rows_per_block), 1, 1, a,
                (unsigned)(2 * dim * sizeof(float)));
}

}  // extern "C"
