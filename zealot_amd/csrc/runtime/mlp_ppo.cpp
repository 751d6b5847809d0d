// mlp_ppo.cpp — the GpuMlp equivalent (zl_mlp) and the whole PPO update
// (zl_ppo) on one device-resident flat parameter buffer.
//
// HBM layout. All parameters of an update live in ONE flat fp32 buffer:
//   actor  w[0] b[0] w[1] b[1] ... | critic w[0] b[0] ... | log_std
// with every tensor start aligned to 64 floats (256 B) and w[l] stored
// [dims[l+1] x ldw] with ldw = dims[l] rounded up to 4, so every GEMM operand
// row is 16-byte aligned for float4 loads (the update's layer-0 weights: up to
// a whole GEMM k-tile when that adds little, see input_align). Gradients and the two Adam moments
// use the same layout, so the optimiser is one flat, vectorised pass (one
// launch for all 2L + 2L + 1 tensors) and the grad-norm clip is a reduction
// over two contiguous ranges. Padding stays zero forever (zero grads give a
// zero Adam update). Activations are batch-major [rows x ld] with ld the
// feature count rounded up to 4.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstddef>
#include <cstring>
#include <string>
#include <vector>

#include "internal.hpp"

namespace zl {

zl_status adv_normalize_into(zl_ctx* c, float* adv, long long n, float* scratch, int nparts,
                             int chunk, const int* guard, float* const* wb);

// Offsets of one MLP's tensors inside the flat buffer.
struct NetLayout {
  std::vector<int> dims;
  int L = 0;
  std::vector<long long> w_off, b_off;
  std::vector<int> ldw;
  long long begin = 0, end = 0;
  long long packed = 0;  // parameter count in the packed (reference) layout

  void build(const int* d, int nd, long long start, int in_align = 4) {
    dims.assign(d, d + nd);
    L = nd - 1;
    w_off.resize(L);
    b_off.resize(L);
    ldw.resize(L);
    begin = start;
    long long cur = start;
    packed = 0;
    for (int l = 0; l < L; ++l) {
      ldw[l] = (int)round_up(dims[l], l == 0 ? in_align : 4);
      w_off[l] = cur;
      cur += round_up((long long)dims[l + 1] * ldw[l], 64);
      b_off[l] = cur;
      cur += round_up(dims[l + 1], 64);
      packed += (long long)dims[l + 1] * dims[l] + dims[l + 1];
    }
    end = cur;
  }
  // Packed (w[0], b[0], w[1], ...; w[l] row-major [out x in]) <-> flat.
  void scatter(const float* packed_src, float* flat) const {
    for (int l = 0; l < L; ++l) {
      const int out = dims[l + 1], in = dims[l];
      for (int o = 0; o < out; ++o)
        std::memcpy(flat + w_off[l] + (long long)o * ldw[l], packed_src + (long long)o * in,
                    (size_t)in * 4);
      packed_src += (long long)out * in;
      std::memcpy(flat + b_off[l], packed_src, (size_t)out * 4);
      packed_src += out;
    }
  }
  void gather(const float* flat, float* packed_dst) const {
    for (int l = 0; l < L; ++l) {
      const int out = dims[l + 1], in = dims[l];
      for (int o = 0; o < out; ++o)
        std::memcpy(packed_dst + (long long)o * in, flat + w_off[l] + (long long)o * ldw[l],
                    (size_t)in * 4);
      packed_dst += (long long)out * in;
      std::memcpy(packed_dst, flat + b_off[l], (size_t)out * 4);
      packed_dst += out;
    }
  }
};

// Row alignment of an update's layer-0 weights and staged observations: a
// whole 32-wide GEMM k-tile when that adds at most 1/8 to the row (123 -> 128
// or 265 -> 288 features), else 4. The staged rows are zero past the features and so are
// the weights' padding columns, so the layer-0 GEMMs can run over the padded
// width (the forward's K, the weight gradient's N) and take the exact-fit
// kernels without changing a result: the extra terms are 0 * 0.
constexpr int kInputTile = 32;
inline int input_align(int d) {
  return round_up(d, kInputTile) * 8 <= (long long)d * 9 ? kInputTile : 4;
}

// Per-row activation and delta buffers of one MLP for up to `rows` rows.
struct NetBuffers {
  int rows = 0;
  std::vector<float*> act;    // act[l], l = 1..L: [rows x ld[l]]
  std::vector<int> ld;        // ld[l] = dims[l] rounded up to 4
  std::vector<float*> delta;  // delta[l], l = 0..L-1: [rows x ld[l+1]] (dL/dz_l)

  zl_status alloc(zl_ctx* c, const NetLayout& nl, int r) {
    rows = r;
    act.assign(nl.L + 1, nullptr);
    delta.assign(nl.L, nullptr);
    ld.assign(nl.L + 1, 0);
    for (int l = 0; l <= nl.L; ++l) ld[l] = (int)round_up(nl.dims[l], 4);
    for (int l = 1; l <= nl.L; ++l)
      ZL_HIP(c, hipMalloc((void**)&act[l], (size_t)r * ld[l] * 4));
    for (int l = 0; l < nl.L; ++l)
      ZL_HIP(c, hipMalloc((void**)&delta[l], (size_t)r * ld[l + 1] * 4));
    return ZL_OK;
  }
  void release() {
    for (float* p : act)
      if (p) hipFree(p);
    for (float* p : delta)
      if (p) hipFree(p);
    act.clear();
    delta.clear();
  }
};

static size_t net_ws_floats(const zl_ctx* c, const NetLayout& nl, int rows) {
  size_t w = 0;
  for (int l = 0; l < nl.L; ++l)
    w = std::max(w, gemm_ws_floats(c, nl.dims[l + 1], nl.dims[l], rows, false, false, zk::kEpiStore));
  return w;
}

// Layer l of GpuMlp::forward (src/bin/biped_train_gpu.rs:364-422): one fused
// GEMM + bias + ELU, linear last layer (zealot-rl/src/net.rs:88-108). kx: the
// layer-0 width, as for wgrad_desc.
static GemmDesc fwd_desc(const NetLayout& nl, const NetBuffers& nb, const float* params,
                         const float* x, int ldx, const int* permx, int rows, const int* guard,
                         int l, int kx = 0) {
  GemmDesc d;
  d.A = l == 0 ? x : nb.act[l];
  d.lda = l == 0 ? ldx : nb.ld[l];
  d.a_kc = true;
  d.permA = l == 0 ? permx : nullptr;
  d.B = params + nl.w_off[l];
  d.ldb = nl.ldw[l];
  d.b_kc = true;
  d.C = nb.act[l + 1];
  d.ldc = nb.ld[l + 1];
  d.M = rows;
  d.N = nl.dims[l + 1];
  d.K = l == 0 && kx > 0 ? kx : nl.dims[l];
  d.K_alg = nl.dims[l];
  d.epi = zk::kEpiBiasN;
  d.bias = params + nl.b_off[l];
  d.act = l < nl.L - 1 ? 1 : 0;
  d.guard = guard;
  return d;
}

// Weight gradient of layer l (GpuMlp::backward, src/bin/biped_train_gpu.rs:423-500,
// math of zealot-rl/src/net.rs:113-140): dW = delta^T . a, split-K over the
// rows with a fixed-order reduction, and the bias gradient as the row sums
// of delta^T fused in. `dl` is dL/dz of the layer. kx > 0: layer 0 runs over
// kx input columns (x and the weights zero past dims[0], kx <= ldw[0]).
static GemmDesc wgrad_desc(const NetLayout& nl, const NetBuffers& nb, float* grads, const float* x,
                           int ldx, const int* permx, int rows, const float* dl, int ldd,
                           const int* guard, int l, int kx = 0) {
  GemmDesc w;
  w.A = dl;
  w.lda = ldd;
  w.a_kc = false;
  w.B = l == 0 ? x : nb.act[l];
  w.ldb = l == 0 ? ldx : nb.ld[l];
  w.b_kc = false;
  w.permB = l == 0 ? permx : nullptr;
  w.C = grads + nl.w_off[l];
  w.ldc = nl.ldw[l];
  w.M = nl.dims[l + 1];
  w.N = l == 0 && kx > 0 ? kx : nl.dims[l];
  w.N_alg = nl.dims[l];
  w.K = rows;
  w.rowsum_out = grads + nl.b_off[l];
  w.guard = guard;
  return w;
}

// Data gradient into layer l-1: delta_{l-1} = (delta_l . W_l) * elu'(a_l),
// ELU' fused into the GEMM epilogue.
static GemmDesc dgrad_desc(const NetLayout& nl, const NetBuffers& nb, const float* params, int rows,
                           const float* dl, int ldd, const int* guard, int l) {
  GemmDesc d;
  d.A = dl;
  d.lda = ldd;
  d.a_kc = true;
  d.B = params + nl.w_off[l];
  d.ldb = nl.ldw[l];
  d.b_kc = false;
  d.C = nb.delta[l - 1];
  d.ldc = nb.ld[l];
  d.M = rows;
  d.N = nl.dims[l];
  d.K = nl.dims[l + 1];
  d.epi = zk::kEpiEluGrad;
  d.Y = nb.act[l];
  d.ldy = nb.ld[l];
  d.guard = guard;
  return d;
}

static zl_status net_forward(zl_ctx* c, const NetLayout& nl, const NetBuffers& nb,
                             const float* params, const float* x, int ldx, const int* permx,
                             int rows, const int* guard, int kx = 0) {
  for (int l = 0; l < nl.L; ++l) {
    const GemmDesc d = fwd_desc(nl, nb, params, x, ldx, permx, rows, guard, l, kx);
    zl_status s = run_gemm(c, d);
    if (s) return s;
  }
  return ZL_OK;
}

// Backward with each weight gradient reduced right after its GEMM. `top` is
// dL/dz of the output layer.
static zl_status net_backward(zl_ctx* c, const NetLayout& nl, const NetBuffers& nb,
                              const float* params, float* grads, const float* x, int ldx,
                              const int* permx, int rows, const float* top, int ld_top,
                              const int* guard, float* ws, size_t ws_floats) {
  for (int l = nl.L - 1; l >= 0; --l) {
    const float* dl = l == nl.L - 1 ? top : nb.delta[l];
    const int ldd = l == nl.L - 1 ? ld_top : nb.ld[l + 1];
    GemmDesc w = wgrad_desc(nl, nb, grads, x, ldx, permx, rows, dl, ldd, guard, l);
    w.ws = ws;
    w.ws_floats = ws_floats;
    zl_status s = run_gemm(c, w);
    if (s) return s;
    if (l > 0) {
      s = run_gemm(c, dgrad_desc(nl, nb, params, rows, dl, ldd, guard, l));
      if (s) return s;
    }
  }
  return ZL_OK;
}

// One net's operands in a paired actor + critic pass.
struct NetView {
  const NetLayout* nl;
  const NetBuffers* nb;
  const float* x;  // layer-0 input rows
  int ldx;
  int kx = 0;      // > 0: x is zero past dims[0] up to kx columns (<= ldw[0])
};

// Forward of both nets, layer by layer, each layer's two GEMMs in one launch
// when the nets have the same depth (otherwise one after the other).
static zl_status pair_forward(zl_ctx* c, const NetView v[2], const float* params,
                              const int* permx, int rows, const int* guard, int layers = -1) {
  if (layers >= 0 && v[0].nl->L == v[1].nl->L) {
    for (int l = 0; l < layers; ++l) {
      GemmDesc d[2];
      for (int i = 0; i < 2; ++i)
        d[i] = fwd_desc(*v[i].nl, *v[i].nb, params, v[i].x, v[i].ldx, permx, rows, guard, l, v[i].kx);
      zl_status s = run_gemm_batch(c, d, 2);
      if (s) return s;
    }
    return ZL_OK;
  }
  if (v[0].nl->L != v[1].nl->L) {
    for (int i = 0; i < 2; ++i) {
      zl_status s = net_forward(c, *v[i].nl, *v[i].nb, params, v[i].x, v[i].ldx, permx, rows, guard,
                                v[i].kx);
      if (s) return s;
    }
    return ZL_OK;
  }
  for (int l = 0; l < v[0].nl->L; ++l) {
    GemmDesc d[2];
    for (int i = 0; i < 2; ++i)
      d[i] = fwd_desc(*v[i].nl, *v[i].nb, params, v[i].x, v[i].ldx, permx, rows, guard, l, v[i].kx);
    zl_status s = run_gemm_batch(c, d, 2);
    if (s) return s;
  }
  return ZL_OK;
}

// Split-K partial regions of every weight gradient of a paired backward
// (they stay alive until the all-layer reduction): region [net][layer] at
// base + off, `size` floats.
struct PartialPlan {
  std::vector<size_t> off[2], size[2];
  size_t total = 0;
  // With fused_head the output layer's region holds zk_head's per-block
  // partials: weights [kHeadMaxBlocks x out x in], then biases [.. x out].
  void build(const zl_ctx* c, const NetLayout* nl[2], int rows, bool fused_head) {
    total = 0;
    for (int i = 0; i < 2; ++i) {
      off[i].assign(nl[i]->L, 0);
      size[i].assign(nl[i]->L, 0);
      for (int l = 0; l < nl[i]->L; ++l) {
        off[i][l] = total;
        const long long M = nl[i]->dims[l + 1], N = nl[i]->dims[l];
        // Layer 0 may run over the padded width ldw[0] (NetView::kx).
        size[i][l] = fused_head && l == nl[i]->L - 1
                         ? (size_t)zk::kHeadMaxBlocks * (M * N + M)
                         : gemm_ws_floats(c, (int)M, (int)N, rows, false, false, zk::kEpiStore);
        if (l == 0)
          size[i][l] = std::max(size[i][l], gemm_ws_floats(c, (int)M, nl[i]->ldw[0], rows, false,
                                                           false, zk::kEpiStore));
        total += round_up((long long)size[i][l], 64);
      }
    }
  }
};

// Backward of both nets with deferred reductions: each layer's weight-gradient
// GEMMs (and data-gradient GEMMs) of the two nets in one launch; the split-K
// reduction of every weight gradient is described in segs[net * L_actor +
// layer] (actor first) for one zk_reduce_all launch afterwards.
static zl_status pair_backward(zl_ctx* c, const NetView v[2], const float* params, float* grads,
                               const int* permx, int rows, const float* const top[2],
                               const int ld_top[2], const int* guard, float* pws,
                               const PartialPlan& pp, zk::ReduceSeg* segs, int depth0 = 0) {
  const int L[2] = {v[0].nl->L, v[1].nl->L};
  const bool paired = L[0] == L[1];
  for (int depth = depth0; depth < std::max(L[0], L[1]); ++depth) {
    GemmDesc w[2], d[2];
    int nw = 0, nd = 0;
    for (int i = 0; i < 2; ++i) {
      const int l = L[i] - 1 - depth;
      if (l < 0) continue;
      const NetLayout& nl = *v[i].nl;
      const NetBuffers& nb = *v[i].nb;
      const float* dl = l == nl.L - 1 ? top[i] : nb.delta[l];
      const int ldd = l == nl.L - 1 ? ld_top[i] : nb.ld[l + 1];
      GemmDesc& q = w[nw++];
      q = wgrad_desc(nl, nb, grads, v[i].x, v[i].ldx, permx, rows, dl, ldd, guard, l, v[i].kx);
      q.ws = pws + pp.off[i][l];
      q.ws_floats = pp.size[i][l];
      q.seg_out = &segs[i * L[0] + l];
      if (l > 0) d[nd++] = dgrad_desc(nl, nb, params, rows, dl, ldd, guard, l);
    }
    // Weight gradients that share a launch with data gradients filling at
    // least three rounds of the CUs (two 128 x 128 tiles per CU each) take
    // half the split-K slices: the data-gradient blocks keep the CUs busy
    // while the longer slices run, and the reduction reads half the
    // partials (the 24,576-row layer-1 backward 225.9 -> 221.6 us and its
    // share of zk_reduce_all ~1.6 us less per minibatch; the layer-2
    // backward, 768 data-gradient tiles, measured 70.8 -> 77.1 us with half
    // and keeps them). ZL_BWD_SPLIT_DIV > 0 sets the divisor for every such
    // layer instead.
    if (paired && nd > 0) {
      long long dg_tiles = 0;
      for (int j = 0; j < nd; ++j) dg_tiles += cdiv(d[j].M, 128) * cdiv(d[j].N, 128);
      int div = c->bwd_split_div;
      if (div == 0) div = dg_tiles >= 6LL * c->cu_count ? 2 : 1;
      if (div > 1)
        for (int j = 0; j < nw; ++j)
          if (w[j].M > 0 && L[j] - 1 - depth > 0)  // a layer with a data gradient
            w[j].splits = std::max(1, gemm_splits(c, w[j].M, w[j].N, w[j].K, w[j].a_kc, w[j].b_kc,
                                                  w[j].epi) / div);
    }
    zl_status s = ZL_OK;
    if (paired) {
      s = run_gemm_bwd(c, w, nw, d, nd);
    } else {
      for (int j = 0; j < nw && !s; ++j) s = run_gemm_batch(c, &w[j], 1);
      for (int j = 0; j < nd && !s; ++j) s = run_gemm_batch(c, &d[j], 1);
    }
    if (s) return s;
  }
  return ZL_OK;
}

static zl_status copy_rows(zl_ctx* c, float* dst, int ldd, const float* src, int lds, int cols,
                           long long rows, const int* perm, int row0, const int* guard,
                           bool zero_pad) {
  zk::CopyRowsArgs a{};
  a.dst = dst;
  a.src = src;
  a.perm = perm;
  a.rows = rows;
  a.cols = cols;
  a.ldd = ldd;
  a.lds = lds;
  a.row0 = row0;
  a.zero_pad = zero_pad ? 1 : 0;
  a.guard = guard;
  return launch(c, K_COPY_ROWS, (unsigned)cdiv(rows * ldd, kThreads), 1, 1, a);
}

// zealot-rl/src/rng.rs:13-31 (only unit() is needed for the shuffle).
struct Lcg {
  uint64_t s;
  explicit Lcg(uint64_t seed) : s(seed | 1ULL) {}
  float unit() {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    return (float)(s >> 40) / (float)(1ULL << 24);
  }
};

}  // namespace zl

using namespace zl;

// ================================================================== zl_mlp

struct zl_mlp {
  zl_ctx* c = nullptr;
  NetLayout nl;
  NetBuffers nb;
  long long nflat = 0;
  float *params = nullptr, *grads = nullptr, *m = nullptr, *v = nullptr;
  float* ws = nullptr;
  size_t ws_floats = 0;
  const float* x = nullptr;
  int ldx = 0, rows = 0;
  // ZL_MLP_FEATURE_MAJOR: the caller's input, output and output gradient are
  // [dim x rows] (GpuMlp's a[0], a[L] and delta[L-1]). The input and the
  // output gradient are transposed into batch-major staging (xs, gtop), the
  // output out of it (out_fm, stride ld_fm), so the GEMMs, their variants and
  // split-K slicing -- and hence every result bit -- are those of the
  // batch-major handle.
  bool fm = false;
  float *xs = nullptr, *gtop = nullptr, *out_fm = nullptr;
  int ldxs = 0, ld_fm = 0;
};

namespace zl {
// dst[j * ldd + i] = src[i * lds + j], i < rows, j < cols (zk_transpose).
static zl_status transpose(zl_ctx* c, float* dst, long long ldd, const float* src, long long lds,
                           long long rows, long long cols) {
  zk::TransposeArgs a{};
  a.src = src;
  a.dst = dst;
  a.rows = rows;
  a.cols = cols;
  a.lds = lds;
  a.ldd = ldd;
  const long long T = zk::kTransposeTile;
  return launch(c, K_TRANSPOSE, (unsigned)cdiv(cols, T), (unsigned)cdiv(rows, T), 1, a);
}
}  // namespace zl

extern "C" {

zl_status zl_mlp_create_ex(zl_ctx* c, const int* dims, int nd, int batch, int flags,
                           zl_mlp** out) {
  if (!c || !dims || !out || nd < 2 || batch < 1) return ZL_ERR_INVALID;
  *out = nullptr;
  if (flags & ~ZL_MLP_FEATURE_MAJOR)
    return fail(c, ZL_ERR_INVALID, "zl_mlp_create_ex: unknown flags 0x%x", flags);
  for (int i = 0; i < nd; ++i)
    if (dims[i] < 1) return fail(c, ZL_ERR_INVALID, "zl_mlp_create: dims[%d] = %d", i, dims[i]);
  zl_mlp* p = new zl_mlp();
  p->c = c;
  p->fm = (flags & ZL_MLP_FEATURE_MAJOR) != 0;
  p->nl.build(dims, nd, 0);
  p->nflat = p->nl.end;
  const size_t bytes = (size_t)p->nflat * 4;
  hipError_t e = hipSuccess;
  for (float** b : {&p->params, &p->grads, &p->m, &p->v}) {
    if (e == hipSuccess) e = hipMalloc((void**)b, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(*b, 0, bytes, c->stream);
  }
  if (p->fm) {
    // Staging rows are zero past the features (never written there).
    const int L = p->nl.L;
    p->ldxs = (int)round_up(dims[0], 4);
    p->ld_fm = (int)round_up(batch, 4);
    const size_t sz[3] = {(size_t)batch * p->ldxs, (size_t)batch * round_up(dims[L], 4),
                          (size_t)dims[L] * p->ld_fm};
    float** dst[3] = {&p->xs, &p->gtop, &p->out_fm};
    for (int i = 0; i < 3; ++i) {
      if (e == hipSuccess) e = hipMalloc((void**)dst[i], sz[i] * 4);
      if (e == hipSuccess) e = hipMemsetAsync(*dst[i], 0, sz[i] * 4, c->stream);
    }
  }
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  zl_status s = e == hipSuccess ? ZL_OK : fail(c, ZL_ERR_HIP, "zl_mlp_create: %s", hipGetErrorString(e));
  if (!s) s = p->nb.alloc(c, p->nl, batch);
  if (!s) {
    p->ws_floats = std::max<size_t>(net_ws_floats(c, p->nl, batch), 1);
    if (hipMalloc((void**)&p->ws, p->ws_floats * 4) != hipSuccess)
      s = fail(c, ZL_ERR_HIP, "zl_mlp_create: scratch alloc failed");
  }
  if (s) {
    zl_mlp_destroy(p);
    return s;
  }
  *out = p;
  return ZL_OK;
}

zl_status zl_mlp_create(zl_ctx* c, const int* dims, int nd, int batch, zl_mlp** out) {
  return zl_mlp_create_ex(c, dims, nd, batch, 0, out);
}

void zl_mlp_destroy(zl_mlp* p) {
  if (!p) return;
  if (p->c && p->c->stream) hipStreamSynchronize(p->c->stream);
  p->nb.release();
  for (float* b : {p->params, p->grads, p->m, p->v, p->ws, p->xs, p->gtop, p->out_fm})
    if (b) hipFree(b);
  delete p;
}

long long zl_mlp_num_params(const zl_mlp* p) { return p ? p->nl.packed : -1; }

static zl_status flat_upload(zl_ctx* c, const NetLayout& nl, long long nflat, float* dev,
                             const float* packed) {
  std::vector<float> host((size_t)nflat, 0.0f);
  nl.scatter(packed, host.data());
  ZL_HIP(c, hipMemcpyAsync(dev, host.data(), host.size() * 4, hipMemcpyHostToDevice, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  return ZL_OK;
}

static zl_status flat_download(zl_ctx* c, const NetLayout& nl, long long nflat, const float* dev,
                               float* packed) {
  std::vector<float> host((size_t)nflat);
  ZL_HIP(c, hipMemcpyAsync(host.data(), dev, host.size() * 4, hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  nl.gather(host.data(), packed);
  return ZL_OK;
}

zl_status zl_mlp_write_weights(zl_mlp* p, const float* packed) {
  if (!p || !packed) return ZL_ERR_INVALID;
  return flat_upload(p->c, p->nl, p->nflat, p->params, packed);
}

zl_status zl_mlp_read_weights(zl_mlp* p, float* packed) {
  if (!p || !packed) return ZL_ERR_INVALID;
  return flat_download(p->c, p->nl, p->nflat, p->params, packed);
}

zl_status zl_mlp_read_grads(zl_mlp* p, float* packed) {
  if (!p || !packed) return ZL_ERR_INVALID;
  return flat_download(p->c, p->nl, p->nflat, p->grads, packed);
}

zl_status zl_mlp_read_moments(zl_mlp* p, float* mh, float* vh) {
  if (!p) return ZL_ERR_INVALID;
  zl_status s = ZL_OK;
  if (mh) s = flat_download(p->c, p->nl, p->nflat, p->m, mh);
  if (!s && vh) s = flat_download(p->c, p->nl, p->nflat, p->v, vh);
  return s;
}

zl_status zl_mlp_write_moments(zl_mlp* p, const float* mh, const float* vh) {
  if (!p) return ZL_ERR_INVALID;
  zl_status s = ZL_OK;
  if (mh) s = flat_upload(p->c, p->nl, p->nflat, p->m, mh);
  if (!s && vh) s = flat_upload(p->c, p->nl, p->nflat, p->v, vh);
  return s;
}

zl_status zl_mlp_forward(zl_mlp* p, const float* x, int ldx, int rows) {
  if (!p) return ZL_ERR_INVALID;
  const int L = p->nl.L;
  // Batch-major x: ldx >= dims[0] (row stride); feature-major: ldx >= rows.
  if (!x || rows < 1 || rows > p->nb.rows || ldx < (p->fm ? rows : p->nl.dims[0]))
    return fail(p->c, ZL_ERR_INVALID, "zl_mlp_forward: rows %d (batch %d), ldx %d", rows,
                p->nb.rows, ldx);
  p->rows = rows;
  if (!p->fm) {
    p->x = x;
    p->ldx = ldx;
    return net_forward(p->c, p->nl, p->nb, p->params, x, ldx, nullptr, rows, nullptr);
  }
  p->x = p->xs;
  p->ldx = p->ldxs;
  zl_status s = transpose(p->c, p->xs, p->ldxs, x, ldx, p->nl.dims[0], rows);
  if (!s) s = net_forward(p->c, p->nl, p->nb, p->params, p->xs, p->ldxs, nullptr, rows, nullptr);
  if (!s) s = transpose(p->c, p->out_fm, p->ld_fm, p->nb.act[L], p->nb.ld[L], rows, p->nl.dims[L]);
  return s;
}

const float* zl_mlp_output(const zl_mlp* p, int* ld_out) {
  if (!p) return nullptr;
  if (p->fm) {
    if (ld_out) *ld_out = p->ld_fm;
    return p->out_fm;
  }
  if (ld_out) *ld_out = p->nb.ld[p->nl.L];
  return p->nb.act[p->nl.L];
}

zl_status zl_mlp_backward(zl_mlp* p, const float* g_out, int ld_g) {
  if (!p) return ZL_ERR_INVALID;
  const int L = p->nl.L;
  if (!g_out || !p->x || ld_g < (p->fm ? p->rows : p->nl.dims[L]))
    return fail(p->c, ZL_ERR_INVALID, "zl_mlp_backward: no forward or bad gradient");
  const float* top = g_out;
  int ld_top = ld_g;
  if (p->fm) {
    top = p->gtop;
    ld_top = p->nb.ld[L];
    zl_status s = transpose(p->c, p->gtop, ld_top, g_out, ld_g, p->nl.dims[L], p->rows);
    if (s) return s;
  }
  return net_backward(p->c, p->nl, p->nb, p->params, p->grads, p->x, p->ldx, nullptr, p->rows,
                      top, ld_top, nullptr, p->ws, p->ws_floats);
}

zl_status zl_mlp_adam(zl_mlp* p, float lr, float bc1, float bc2) {
  if (!p) return ZL_ERR_INVALID;
  return zl_adam_step(p->c, p->params, p->grads, p->m, p->v, (size_t)p->nflat, lr, 0.9f, 0.999f,
                      1e-8f, bc1, bc2);
}

}  // extern "C"

// ================================================================== zl_ppo

struct zl_ppo {
  zl_ctx* c = nullptr;
  NetLayout actor, critic;
  long long ls_off = 0;
  int A = 0;
  long long nflat = 0;
  float *params = nullptr, *grads = nullptr, *m = nullptr, *v = nullptr;
  NetBuffers ab, cb;
  int mb_cap = 0;
  // The output layers and the losses run as one zk_head launch (last hidden
  // widths <= kHeadMaxHidden, A <= kHeadMaxActions, equal depths;
  // ZL_FUSED_HEAD=0 turns it off). head_fwd: with two or more hidden layers
  // that launch also computes the last hidden layer's forward, tile by tile
  // (zk_head_fwd*), when a minibatch takes one tile per block
  // (ZL_FUSED_HEAD=1 keeps that layer a GEMM launch of its own).
  bool fused_head = false;
  bool head_fwd = false;
  // Reduction partials.
  float* gls_part = nullptr;  // [nb x A]
  float* astat_part = nullptr;
  float* vstat_part = nullptr;
  float* sq_part = nullptr;  // grad-norm partials, one per zk_reduce_all block
  int sq_cap = 0;
  float* kl_part = nullptr;
  float* adv_part = nullptr;
  int nb_cap = 0;
  static constexpr int kAdvChunk = 4096;
  // Split-K partials of every weight gradient of a minibatch step, alive
  // until the all-layer reduction (regions laid out for `pplan_rows` rows).
  float* pws = nullptr;
  size_t pws_cap = 0;
  PartialPlan pplan;
  size_t adv_part_cap = 0;
  // Device scalars of an update followed by the caller's batch pointers
  // (UpdateIn), uploaded together before every update.
  zk::DevState* dstate = nullptr;
  zk::BatchPtrs* bptrs = nullptr;
  float* ls_old = nullptr;
  float* stat_out = nullptr;  // [8] scratch for zl_ppo_minibatch_grads
  // The staged batch (zk_stage): actor obs [n x odp], critic obs [n x cdp],
  // action [n x A], mean_old [n x A], then logp_old, value_old, adv, ret [n].
  float* stg[8] = {};
  size_t stg_cap[8] = {};
  // Observation staging of the rollout step and the chunked forwards
  // (padded, 16-byte aligned rows) and shuffle orders.
  float* obs_pad = nullptr;
  size_t obs_pad_floats = 0;
  float* cobs_pad = nullptr;
  size_t cobs_pad_floats = 0;
  int* perm = nullptr;
  size_t perm_cap = 0;
  // Shuffle orders of ActorCritic::update in pinned host memory, two
  // buffers: one uploaded for the update in flight, the other filled with the
  // next update's orders (its Adam step count is known: one step per
  // minibatch) while the device runs this one. A buffer is used only if its
  // key matches the call.
  struct ShuffleBuf {
    int* h = nullptr;
    size_t cap = 0;  // ints
    long long n = -1;
    int epochs = 0, minibatches = 0, t = -1;
  };
  ShuffleBuf shuf[2];
  int shuf_cur = 0;
  zk::DevState hstate{};
  // Bumped whenever a device buffer of this handle is reallocated: a captured
  // graph is only replayed while every buffer it references is still alive.
  unsigned long long gen = 0;
  // zk_policy's fragment-major copy of the weights of each net that fits it
  // (zk_policy_pack), rewritten after every change of the parameters
  // (zl_ppo_create, zl_ppo_set_params and so zl_ppo_load, the end of every
  // update, eager or captured), so that it matches them at every point of
  // the stream where a call that reads it runs.
  float* polw = nullptr;
  long long polw_off[2][zk::kPolicyMaxLayers] = {};
  bool polw_net[2] = {false, false};
  zk::PolicyPackArgs pack{};
  // Captured update graph and the signature it was captured for.
  hipGraphExec_t gexec = nullptr;
  std::string gkey;
  long long captures = 0;
  double capture_ms = 0.0;
};

namespace {

// zk_policy: below this many rows a forward runs as one launch (each block
// reads every weight once from L2, so the weight traffic grows with the row
// blocks; the layer GEMMs take larger batches).
constexpr long long kPolicyFusedRows = 8192;

// Whether a net fits zk_policy: at most kPolicyMaxLayers layers, hidden widths
// multiples of 16 up to kPolicyMaxWidth, input width up to kPolicyMaxWidth
// with its 16-padded width inside the layer-0 weight rows, at most 32 outputs,
// 16-byte aligned weight rows.
static bool policy_fits(const zl_ppo* p, const NetLayout& nl) {
  if (nl.L < 1 || nl.L > zk::kPolicyMaxLayers || nl.dims[0] > zk::kPolicyMaxWidth ||
      nl.dims[nl.L] > 32 || nl.ldw[0] < round_up(nl.dims[0], 16))
    return false;
  for (int l = 1; l < nl.L; ++l)
    if (nl.dims[l] % 16 != 0 || nl.dims[l] > zk::kPolicyMaxWidth) return false;
  for (int l = 0; l < nl.L; ++l)
    if (nl.w_off[l] % 4 != 0 || nl.ldw[l] % 4 != 0) return false;
  return ((uintptr_t)p->params & 15) == 0;
}

// zk_policy_pack's segments for the nets that fit zk_policy and the size of
// their packed copy in floats: per layer, ceil(N / 16) tiles x ceil(K / 16)
// chunks x 256 floats (K the layer's input width).
static long long policy_layout(zl_ppo* p) {
  zk::PolicyPackArgs& a = p->pack;
  a = zk::PolicyPackArgs{};
  long long floats = 0;
  for (int net = 0; net < 2; ++net) {
    const NetLayout& nl = net ? p->critic : p->actor;
    p->polw_net[net] = policy_fits(p, nl);
    if (!p->polw_net[net]) continue;
    for (int l = 0; l < nl.L; ++l) {
      zk::PolicyPackSeg& g = a.seg[a.nseg++];
      g.src = nl.w_off[l];
      g.dst = floats;
      g.q0 = floats / 4;
      g.ldw = nl.ldw[l];
      g.N = nl.dims[l + 1];
      g.K = nl.dims[l];
      g.kc = (int)cdiv(nl.dims[l], 16);
      p->polw_off[net][l] = floats;
      floats += cdiv(g.N, 16) * g.kc * 256;
    }
  }
  a.nq = floats / 4;
  return floats;
}

// Rewrite zk_policy's copy of the weights from the parameters (stream-ordered
// after whatever wrote them).
static zl_status policy_pack(zl_ppo* p) {
  if (p->pack.nseg == 0) return ZL_OK;
  p->pack.params = p->params;
  p->pack.dst = p->polw;
  return launch(p->c, K_POLICY_PACK, (unsigned)cdiv(p->pack.nq, kThreads), 1, 1, p->pack);
}

// Grow a device buffer of the handle (outside graph capture: may synchronize).
// A reallocation bumps the handle's buffer generation, which is part of the
// captured update graph's key.
zl_status grow(zl_ppo* pp, void** p, size_t* cap, size_t bytes) {
  zl_ctx* c = pp->c;
  if (bytes <= *cap) return ZL_OK;
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  pp->gen += 1;
  if (*p) ZL_HIP(c, hipFree(*p));
  *p = nullptr;
  *cap = 0;
  ZL_HIP(c, hipMalloc(p, bytes));
  *cap = bytes;
  return ZL_OK;
}

// Host image of the device block at zl_ppo::dstate.
struct UpdateIn {
  zk::DevState st;
  zk::BatchPtrs ptrs;
};

// Lay out the weight-gradient partial regions for minibatches of `rows` rows
// and grow their buffer (outside graph capture: may synchronize).
zl_status ensure_partials(zl_ppo* p, int rows) {
  const NetLayout* nls[2] = {&p->actor, &p->critic};
  p->pplan.build(p->c, nls, rows, p->fused_head);
  size_t cap = p->pws_cap * 4;
  zl_status s = grow(p, (void**)&p->pws, &cap, p->pplan.total * 4 + 4);
  p->pws_cap = cap / 4;
  return s;
}

// Backward of both nets for one minibatch plus the all-layer reduction with
// the grad-norm partials; nsq / nsq_a receive the partial counts (all, actor).
// With `tail`, the reduction launch also runs the minibatch tail. head_blocks
// (actor) / critic_blocks: zk_head's partial counts per net (0: no zk_head).
zl_status backward_and_reduce(zl_ppo* p, const NetView v[2], const int* permx, int rows,
                              const int* guard, int* nsq, int* nsq_a, int head_blocks,
                              int critic_blocks, const zk::FinalizeArgs* tail) {
  zl_ctx* c = p->c;
  const int La = p->actor.L, Lc = p->critic.L;
  const float* top[2] = {p->ab.delta[La - 1], p->cb.delta[Lc - 1]};
  const int ldt[2] = {p->ab.ld[La], p->cb.ld[Lc]};
  zk::ReduceSeg segs[zk::kMaxReduceSegs];
  // With the fused head, zk_head has produced dL/dz of the last hidden layers
  // and the output layers' gradient partials: the backward starts one layer
  // down and the output layers' segments describe those partials.
  zl_status s = pair_backward(c, v, p->params, p->grads, permx, rows, top, ldt, guard, p->pws,
                              p->pplan, segs, head_blocks > 0 ? 1 : 0);
  if (s) return s;
  if (head_blocks > 0) {
    for (int i = 0; i < 2; ++i) {
      const NetLayout& nl = i == 0 ? p->actor : p->critic;
      const int l = nl.L - 1;
      const long long M = nl.dims[l + 1], N = nl.dims[l];
      float* part = p->pws + p->pplan.off[i][l];
      zk::ReduceSeg& r = segs[i * La + l];
      r = zk::ReduceSeg{};
      r.part = part;
      r.rowpart = part + (size_t)zk::kHeadMaxBlocks * M * N;
      r.out = p->grads + nl.w_off[l];
      r.rowout = p->grads + nl.b_off[l];
      r.mn = M * N;
      r.cols = (int)N;
      r.ldo = nl.ldw[l];
      r.rows = (int)M;
      r.splits = i == 0 ? head_blocks : critic_blocks;
    }
  }
  zk::ReduceSeg lay[zk::kMaxReduceSegs];
  std::copy(segs, segs + La + Lc, lay);
  const int blocks = reduce_all_layout(lay, La + Lc);
  if (blocks + 1 > p->sq_cap)
    return fail(c, ZL_ERR_INVALID, "grad-norm partials: %d blocks > capacity %d", blocks + 1,
                p->sq_cap);
  *nsq = blocks;
  *nsq_a = lay[La].blk0;
  return launch_reduce_all(c, segs, La + Lc, p->sq_part, guard, tail);
}

// Per-epoch Fisher-Yates orders of ActorCritic::update for Adam step count t
// (zealot-rl/src/ppo.rs:357-363: Lcg::new(t_logstd + 1), and t_logstd
// advances once per minibatch, so epoch e starts at t + e * minibatches),
// into sb (pinned, grown as needed; the allocation is the only failure).
static hipError_t shuffle_orders(zl_ppo::ShuffleBuf& sb, long long n, int epochs, int minibatches,
                                 int t) {
  const size_t need = (size_t)epochs * (size_t)n;
  sb.n = -1;
  if (sb.cap < need) {
    if (sb.h) hipHostFree(sb.h);
    sb.h = nullptr;
    sb.cap = 0;
    hipError_t e = hipHostMalloc((void**)&sb.h, std::max<size_t>(need, 1) * 4, hipHostMallocDefault);
    if (e != hipSuccess) {
      sb.h = nullptr;
      return e;
    }
    sb.cap = need;
  }
  for (int e = 0; e < epochs; ++e) {
    int* order = sb.h + (size_t)e * n;
    for (long long i = 0; i < n; ++i) order[i] = (int)i;
    Lcg sh((uint64_t)(t + e * minibatches) + 1);
    for (long long i = n - 1; i >= 1; --i) {
      size_t j = (size_t)(sh.unit() * (float)(i + 1));
      std::swap(order[i], order[std::min<long long>((long long)j, i)]);
    }
  }
  sb.n = n;
  sb.epochs = epochs;
  sb.minibatches = minibatches;
  sb.t = t;
  return hipSuccess;
}

// Loss-partial and grad-norm-partial counts of one minibatch pass.
struct PassCounts {
  int nb_a = 0, nb_v = 0, nsq = 0, nsq_a = 0;
};

// One minibatch: forward of both nets, the PPO losses, backward, and the
// all-layer reduction with the grad-norm partials (the accumulation of
// zealot-rl/src/ppo.rs:406-462 before clip / Adam). `px` gathers the
// layer-0 rows; samples of the batch are perm[row0 + r] (or row0 + r). With
// `head_kl`, zk_head also writes the per-component KL sums of this minibatch
// there. With `tail` (its loss-partial counts are filled in here), the
// reduction launch also runs the minibatch's scalar tail.
zl_status minibatch_pass(zl_ppo* p, const NetView v[2], const int* px, const int* perm, int row0,
                         int rows, const zl_batch* b, const zl_ppo_config* cfg, float scale,
                         const int* guard, PassCounts* pc, float* head_kl = nullptr,
                         zk::FinalizeArgs* tail = nullptr) {
  zl_ctx* c = p->c;
  const int La = p->actor.L, Lc = p->critic.L, A = p->A;
  const long long tiles = cdiv(rows, zk::kHeadRows);
  const long long tpb = cdiv(tiles, zk::kHeadMaxBlocks);
  // The last hidden layer's forward inside zk_head: one tile per block, and
  // operands that the GEMM tile reads as aligned float4 rows.
  bool hfwd = p->fused_head && p->head_fwd && tpb == 1;
  bool hfwd_exact = hfwd && rows % zk::kHeadRows == 0;
  for (int i = 0; i < 2 && hfwd; ++i) {
    const NetLayout& nl = i == 0 ? p->actor : p->critic;
    const NetBuffers& nb = i == 0 ? p->ab : p->cb;
    const int l = nl.L - 2;
    const float* w2 = p->params + nl.w_off[l];
    hfwd = ((uintptr_t)nb.act[l] & 15) == 0 && ((uintptr_t)w2 & 15) == 0 && nb.ld[l] % 4 == 0 &&
           nl.ldw[l] % 4 == 0;
    hfwd_exact = hfwd_exact && nl.dims[l + 1] == zk::kHeadMaxHidden && nl.dims[l] % 32 == 0;
  }
  zl_status s = pair_forward(c, v, p->params, px, rows, guard,
                             p->fused_head ? (hfwd ? La - 2 : La - 1) : -1);
  if (s) return s;
  int head_blocks = 0, critic_blocks = 0;
  if (p->fused_head) {
    head_blocks = (int)cdiv(tiles, tpb);
    // A critic tile is about a third of an actor tile's work: when the actor
    // takes one tile per block and leaves workgroup slots free (two per CU),
    // the critic takes its tiles in that many blocks, up to three tiles each
    // (each tile's loads in flight during the previous one), so both nets
    // finish in one round; otherwise it is laid out like the actor. With
    // the forward inside, a tile of either net is mostly that GEMM: one tile
    // per block for both (two or three critic tiles per block measured 2-12 %
    // slower).
    const int slots = 2 * c->cu_count;
    long long ctiles = tpb;
    if (!hfwd && tpb == 1 && head_blocks < slots)
      ctiles = std::min<long long>(3, cdiv(tiles, slots - head_blocks));
    critic_blocks = (int)cdiv(tiles, ctiles);
    zk::HeadArgs h{};
    double fwd_flops = 0.0;
    for (int i = 0; i < 2; ++i) {
      const NetLayout& nl = i == 0 ? p->actor : p->critic;
      const NetBuffers& nb = i == 0 ? p->ab : p->cb;
      const int l = nl.L - 1;
      zk::HeadNet& q = h.net[i];
      q.x = nb.act[l];
      q.ldx = nb.ld[l];
      q.w = p->params + nl.w_off[l];
      q.ldw = nl.ldw[l];
      q.b = p->params + nl.b_off[l];
      q.out = nb.act[l + 1];
      q.ldo = nb.ld[l + 1];
      q.dz = nb.delta[l - 1];
      q.ldz = nb.ld[l];
      q.H = nl.dims[l];
      q.wpart = p->pws + p->pplan.off[i][l];
      q.bpart = q.wpart + (size_t)zk::kHeadMaxBlocks * nl.dims[l + 1] * nl.dims[l];
      if (hfwd) {
        q.x2 = nb.act[l - 1];
        q.ldx2 = nb.ld[l - 1];
        q.w2 = p->params + nl.w_off[l - 1];
        q.ldw2 = nl.ldw[l - 1];
        q.b2 = p->params + nl.b_off[l - 1];
        q.k2 = nl.dims[l - 1];
        fwd_flops += 2.0 * rows * nl.dims[l] * (double)nl.dims[l - 1];
      }
    }
    h.action = b->action;
    h.ldact = b->ld_action;
    h.logp_old = b->logp_old;
    h.adv = b->adv;
    h.mean_old = b->mean_old;
    h.ldmo = b->ld_mean_old;
    h.log_std = p->params + p->ls_off;
    h.value_old = b->value_old;
    h.ret = b->ret;
    h.perm = perm;
    h.row0 = row0;
    h.rows = rows;
    h.A = A;
    h.tiles_per_block = (int)tpb;
    h.critic_blocks = critic_blocks;
    h.critic_tiles = (int)ctiles;
    h.clip = cfg->clip;
    h.entropy_coef = cfg->entropy_coef;
    h.value_coef = cfg->value_coef;
    h.scale = scale;
    h.gls_part = p->gls_part;
    h.astat_part = p->astat_part;
    h.vstat_part = p->vstat_part;
    h.kl_part = head_kl;
    h.guard = guard;
    c->pending_flops = fwd_flops;  // the layer GEMM work inside (timing)
    if ((s = launch(c, hfwd ? (hfwd_exact ? K_HEAD_FWD_X : K_HEAD_FWD) : K_HEAD, (unsigned)head_blocks,
                    1, 2, h, 0, zk::kHeadThreads)))
      return s;
    pc->nb_a = head_blocks;
    pc->nb_v = critic_blocks;
  } else {
    const LossShape lsh = actor_loss_shape(rows, A);
    zk::ActorLossArgs al{};
    al.mean = p->ab.act[La];
    al.ldm = p->ab.ld[La];
    al.action = b->action;
    al.ldact = b->ld_action;
    al.adv = b->adv;
    al.logp_old = b->logp_old;
    al.mean_old = b->mean_old;
    al.ldmo = b->ld_mean_old;
    al.cm = al.cact = al.cmo = al.cdd = 1;
    al.log_std = p->params + p->ls_off;
    al.perm = perm;
    al.row0 = row0;
    al.rows = rows;
    al.A = A;
    al.delta = p->ab.delta[La - 1];
    al.ldd = p->ab.ld[La];
    al.gls_part = p->gls_part;
    al.stat_part = p->astat_part;
    al.guard = guard;
    al.clip = cfg->clip;
    al.entropy_coef = cfg->entropy_coef;
    al.scale = scale;
    al.rows_per_block = lsh.rows_per_block;
    al.group = lsh.group;
    if ((s = launch(c, lsh.kernel, (unsigned)lsh.blocks, 1, 1, al, 0, zk::kLossThreads))) return s;
    const int nbv = (int)cdiv(rows, kThreads);
    zk::ValueLossArgs vl{};
    vl.v = p->cb.act[Lc];
    vl.ldv = p->cb.ld[Lc];
    vl.value_old = b->value_old;
    vl.ret = b->ret;
    vl.perm = perm;
    vl.row0 = row0;
    vl.rows = rows;
    vl.delta = p->cb.delta[Lc - 1];
    vl.ldd = p->cb.ld[Lc];
    vl.stat_part = p->vstat_part;
    vl.guard = guard;
    vl.clip = cfg->clip;
    vl.value_coef = cfg->value_coef;
    vl.scale = scale;
    if ((s = launch(c, K_VALUE_LOSS, (unsigned)nbv, 1, 1, vl))) return s;
    pc->nb_a = lsh.blocks;
    pc->nb_v = nbv;
  }
  if (tail) {
    tail->nb_a = pc->nb_a;
    tail->nb_v = pc->nb_v;
  }
  return backward_and_reduce(p, v, px, rows, guard, &pc->nsq, &pc->nsq_a, head_blocks, critic_blocks,
                             tail);
}

struct Plan {
  int mode, mb, n_mb, epochs;
  long long n;
  bool share_cobs, shuffle;
  const float* X;
  int ldx;
  const float* XC;
  int ldxc;
  zl_batch sb;  // the staged batch: batch-major rows in the handle's buffers
  zk::StageArgs stage;
  int stage_blocks;
  zk::PpoParams pp;
};

// A batch field with element (sample i, feature k) at i * ld + k (batch-major)
// or k * ld + i (feature-major) over n samples of `cols` features.
bool field_ok(long long n, int cols, int ld, bool fm) { return fm ? ld >= n : ld >= cols; }

zl_status check_batch(zl_ppo* p, const zl_batch* b, const char* who) {
  zl_ctx* c = p->c;
  if (!b->obs || !b->critic_obs || !b->action || !b->logp_old || !b->value_old || !b->adv ||
      !b->ret)
    return fail(c, ZL_ERR_INVALID, "%s: null batch pointer", who);
  if (b->n < 0 || b->n > (1LL << 31) - 1)
    return fail(c, ZL_ERR_INVALID, "%s: n = %lld out of range", who, b->n);
  const unsigned fm = b->feature_major;
  if (fm & ~(ZL_FM_OBS | ZL_FM_CRITIC_OBS | ZL_FM_ACTION | ZL_FM_MEAN_OLD))
    return fail(c, ZL_ERR_INVALID, "%s: unknown feature_major bits 0x%x", who, fm);
  if (!field_ok(b->n, p->actor.dims[0], b->ld_obs, fm & ZL_FM_OBS) ||
      !field_ok(b->n, p->critic.dims[0], b->ld_critic_obs, fm & ZL_FM_CRITIC_OBS) ||
      !field_ok(b->n, p->A, b->ld_action, fm & ZL_FM_ACTION) ||
      (b->mean_old && !field_ok(b->n, p->A, b->ld_mean_old, fm & ZL_FM_MEAN_OLD)))
    return fail(c, ZL_ERR_INVALID, "%s: a stride is smaller than the row (or, feature-major, than n)",
                who);
  return ZL_OK;
}

// Lay out the staged copy of `rows` batch samples (source sample perm[row0 + r],
// or row0 + r) in the handle's buffers, growing them as needed: the zk_stage
// launch reading the caller's pointers from p->bptrs, and the staged batch
// view (batch-major rows; observation rows padded to the layer-0 weight rows
// and zero-filled, 16-byte aligned for the layer-0 GEMM loads).
zl_status plan_stage(zl_ppo* p, const zl_batch* b, long long rows, const int* perm, long long row0,
                     zk::StageArgs* st, int* blocks, zl_batch* sb, bool* share_out) {
  const int od = p->actor.dims[0], cd = p->critic.dims[0], A = p->A;
  const int odp = p->actor.ldw[0], cdp = p->critic.ldw[0];  // zero-filled past od / cd
  const unsigned fm = b->feature_major;
  const bool share = b->critic_obs == b->obs && b->ld_critic_obs == b->ld_obs && od == cd &&
                     ((fm & ZL_FM_OBS) != 0) == ((fm & ZL_FM_CRITIC_OBS) != 0);
  const bool has_mo = b->mean_old != nullptr;
  const long long need[8] = {rows * odp, share ? 0 : rows * cdp, rows * A, has_mo ? rows * A : 0,
                             rows, rows, rows, rows};
  for (int i = 0; i < 8; ++i) {
    if (need[i] <= 0) continue;
    zl_status s = grow(p, (void**)&p->stg[i], &p->stg_cap[i], (size_t)need[i] * 4);
    if (s) return s;
  }
  *st = zk::StageArgs{};
  st->ptrs = p->bptrs;
  st->perm = perm;
  st->rows = rows;
  st->row0 = row0;
  int blk = 0, nj = 0;
  auto mat = [&](int slot, int cols, int ld, int ldd, bool f) {
    zk::StageJob& j = st->job[nj++];
    j.dst = p->stg[slot];
    j.ld = ld;
    j.cols = cols;
    j.ldd = ldd;
    j.fm = f ? 1 : 0;
    j.slot = slot;
    j.vec = 0;
    j.tiles_c = (int)cdiv(ldd, zk::kStageCols);
    j.blk0 = blk;
    j.blocks = (int)(cdiv(rows, zk::kStageRows) * j.tiles_c);
    blk += j.blocks;
  };
  mat(0, od, b->ld_obs, odp, fm & ZL_FM_OBS);
  if (!share) mat(1, cd, b->ld_critic_obs, cdp, fm & ZL_FM_CRITIC_OBS);
  mat(2, A, b->ld_action, A, fm & ZL_FM_ACTION);
  if (has_mo) mat(3, A, b->ld_mean_old, A, fm & ZL_FM_MEAN_OLD);
  for (int v = 0; v < 4; ++v) {
    zk::StageJob& j = st->job[nj++];
    j.dst = p->stg[4 + v];
    j.ld = 1;
    j.cols = 1;
    j.ldd = 1;
    j.slot = v;
    j.vec = 1;
    j.blk0 = blk;
    j.blocks = (int)cdiv(rows, zk::kStageVec);
    blk += j.blocks;
  }
  st->njobs = nj;
  *blocks = rows > 0 ? blk : 0;
  *sb = zl_batch{};
  sb->n = rows;
  sb->obs = p->stg[0];
  sb->ld_obs = odp;
  sb->critic_obs = share ? p->stg[0] : p->stg[1];
  sb->ld_critic_obs = share ? odp : cdp;
  sb->action = p->stg[2];
  sb->ld_action = A;
  sb->mean_old = has_mo ? p->stg[3] : nullptr;
  sb->ld_mean_old = A;
  sb->logp_old = p->stg[4];
  sb->value_old = p->stg[5];
  sb->adv = p->stg[6];
  sb->ret = p->stg[7];
  *share_out = share;
  return ZL_OK;
}

zk::BatchPtrs batch_ptrs(const zl_batch* b) {
  zk::BatchPtrs h{};
  h.mat[0] = b->obs;
  h.mat[1] = b->critic_obs;
  h.mat[2] = b->action;
  h.mat[3] = b->mean_old;
  h.vec[0] = b->logp_old;
  h.vec[1] = b->value_old;
  h.vec[2] = b->adv;
  h.vec[3] = b->ret;
  h.adv_out = b->adv;
  return h;
}

zl_status enqueue_update(zl_ppo* p, const zl_ppo_config* cfg, const Plan& pl) {
  zl_ctx* c = p->c;
  // Kernels after a KL early stop are skipped through the device flag
  // `active`; only the early stop clears it, so without one the kernels get
  // no flag and skip the dependent load of it at their start.
  const int* guard = pl.pp.early_stop ? &p->dstate->active : nullptr;
  const int A = p->A;
  const zl_batch* b = &pl.sb;
  zl_status s = launch(c, K_STAGE, (unsigned)pl.stage_blocks, 1, 1, pl.stage);
  if (s) return s;
  if (cfg->normalize_adv) {
    // In place in the staged copy, and written back to the caller's adv
    // (ActorCritic::update normalises the batch it was given, ppo.rs:343-348).
    const int nparts = (int)cdiv(pl.n, zl_ppo::kAdvChunk);
    s = adv_normalize_into(c, b->adv, pl.n, p->adv_part, nparts, zl_ppo::kAdvChunk, guard,
                           &p->bptrs->adv_out);
    if (s) return s;
  }
  const int La = p->actor.L;
  const int nb = (int)cdiv(pl.mb, kThreads);
  const float* log_std = p->params + p->ls_off;
  const bool trainer_kl = pl.mode == ZL_SEMANTICS_GPU_TRAINER && b->mean_old != nullptr;
  // The per-epoch KL of the last minibatch comes from zk_head's per-component
  // sums when the output layers are fused, else from zk_kl.
  const bool head_kl = trainer_kl && p->fused_head;
  for (int e = 0; e < pl.epochs; ++e) {
    if (e == 0) {  // later epochs are opened by the previous zk_epoch_end
      zk::EpochBeginArgs eb{};
      eb.st = p->dstate;
      eb.guard = guard;
      eb.pp = pl.pp;
      if ((s = launch(c, K_EPOCH_BEGIN, 1, 1, 1, eb))) return s;
    }
    const int* perm_e = pl.shuffle ? p->perm + (size_t)e * pl.n : nullptr;
    int nb_kl = nb;
    for (int k = 0; k < pl.n_mb; ++k) {
      const int row0 = k * pl.mb;
      const int* px = perm_e ? perm_e + row0 : nullptr;
      const float* xa = perm_e ? pl.X : pl.X + (size_t)row0 * pl.ldx;
      const float* xc = perm_e ? pl.XC : pl.XC + (size_t)row0 * pl.ldxc;
      const NetView v[2] = {{&p->actor, &p->ab, xa, pl.ldx, pl.ldx},
                            {&p->critic, &p->cb, xc, pl.ldxc, pl.ldxc}};
      float* hkl = head_kl && k == pl.n_mb - 1 ? p->kl_part : nullptr;
      // The step's scalar tail (statistics, log_std gradient, Adam step count,
      // lr rule) runs as the last block of the gradient reduction; zk_adam
      // takes the clip scales from the squared-norm partials itself.
      zk::FinalizeArgs fz{};
      fz.st = p->dstate;
      fz.gls_part = p->gls_part;
      fz.astat_part = p->astat_part;
      fz.vstat_part = p->vstat_part;
      fz.sq_part = p->sq_part;
      fz.log_std = log_std;
      fz.g_logstd = p->grads + p->ls_off;
      fz.pp = pl.pp;
      PassCounts pc;
      if ((s = minibatch_pass(p, v, px, perm_e, row0, pl.mb, b, cfg, pl.pp.scale, guard, &pc, hkl,
                              &fz)))
        return s;
      if (hkl) nb_kl = pc.nb_a;
      zk::AdamArgs ad{};
      ad.p = p->params;
      ad.g = p->grads;
      ad.m = p->m;
      ad.v = p->v;
      ad.st = p->dstate;
      ad.guard = guard;
      ad.n = p->nflat;
      ad.end_a = p->critic.begin;
      ad.end_c = p->ls_off;
      ad.beta1 = pl.pp.beta1;
      ad.beta2 = pl.pp.beta2;
      ad.eps = pl.pp.eps;
      ad.clamp_ls = pl.pp.clamp_ls;
      ad.sq_part = p->sq_part;
      ad.nsq_a = pc.nsq_a;
      ad.nsq = pc.nsq;
      ad.clip = pl.pp.mode == 0 ? 1 : 2;
      ad.max_grad_norm = pl.pp.max_grad_norm;
      if ((s = launch(c, K_ADAM, (unsigned)cdiv(p->nflat, 4 * kThreads), 1, 1, ad))) return s;
    }
    if (trainer_kl && !head_kl) {  // src/bin/biped_train_gpu.rs:1469-1492 (last minibatch)
      zk::KlArgs kl{};
      kl.mean = p->ab.act[La];
      kl.ldm = p->ab.ld[La];
      kl.mean_old = b->mean_old;
      kl.ldmo = b->ld_mean_old;
      kl.log_std = log_std;
      kl.log_std_old = p->ls_old;
      kl.perm = nullptr;
      kl.row0 = (pl.n_mb - 1) * pl.mb;
      kl.rows = pl.mb;
      kl.A = A;
      kl.part = p->kl_part;
      kl.guard = guard;
      if ((s = launch(c, K_KL, (unsigned)nb, 1, 1, kl))) return s;
    }
    zk::EpochEndArgs ee{};
    ee.st = p->dstate;
    ee.kl_part = trainer_kl ? p->kl_part : nullptr;
    ee.log_std = log_std;
    ee.log_std_old = p->ls_old;
    ee.active = &p->dstate->active;
    ee.pp = pl.pp;
    ee.nkl = nb_kl;
    ee.kl_form = head_kl ? 1 : 0;
    ee.begin_next = e + 1 < pl.epochs ? 1 : 0;
    if ((s = launch(c, K_EPOCH_END, 1, 1, 1, ee, 0, zk::kFinalizeThreads))) return s;
  }
  if (pl.mode == ZL_SEMANTICS_GPU_TRAINER && cfg->clamp_log_std) {
    // src/bin/biped_train_gpu.rs:1529-1541, after the epoch loop (even after an early stop).
    zk::ClampArgs cl{};
    cl.x = p->params + p->ls_off;
    cl.n = A;
    cl.lo = -1.6f;
    cl.hi = 0.0f;
    if ((s = launch(c, K_CLAMP, 1, 1, 1, cl))) return s;
  }
  // The rollout step's copy of the updated weights (unguarded: it runs after
  // an early stop too).
  return policy_pack(p);
}

}  // namespace

extern "C" {

zl_status zl_ppo_create(zl_ctx* c, const int* adims, int na, const int* cdims, int nc, int mb,
                        zl_ppo** out) {
  if (!c || !adims || !cdims || !out || na < 2 || nc < 2 || mb < 1) return ZL_ERR_INVALID;
  *out = nullptr;
  for (int i = 0; i < na; ++i)
    if (adims[i] < 1) return fail(c, ZL_ERR_INVALID, "zl_ppo_create: actor dims[%d] = %d", i, adims[i]);
  for (int i = 0; i < nc; ++i)
    if (cdims[i] < 1) return fail(c, ZL_ERR_INVALID, "zl_ppo_create: critic dims[%d] = %d", i, cdims[i]);
  if (cdims[nc - 1] != 1)
    return fail(c, ZL_ERR_INVALID, "zl_ppo_create: critic must output a scalar");  // ppo.rs:242-246
  if (adims[na - 1] > 48)
    return fail(c, ZL_ERR_INVALID, "zl_ppo_create: action dim %d > 48", adims[na - 1]);
  if ((na - 1) + (nc - 1) > zk::kMaxReduceSegs)
    return fail(c, ZL_ERR_INVALID, "zl_ppo_create: more than %d layers in actor + critic",
                zk::kMaxReduceSegs);
  zl_ppo* p = new zl_ppo();
  p->c = c;
  p->actor.build(adims, na, 0, input_align(adims[0]));
  p->critic.build(cdims, nc, p->actor.end, input_align(cdims[0]));
  p->A = adims[na - 1];
  p->ls_off = p->critic.end;
  p->nflat = p->ls_off + round_up(p->A, 64);
  p->mb_cap = mb;
  {
    const int ha = adims[na - 2], hc = cdims[nc - 2];
    const char* env = getenv("ZL_FUSED_HEAD");
    p->fused_head = na == nc && na >= 3 && ha <= zk::kHeadMaxHidden && hc <= zk::kHeadMaxHidden &&
                    p->A <= zk::kHeadMaxActions && !(env && atoi(env) == 0);
    p->head_fwd = p->fused_head && na >= 4 && !(env && atoi(env) == 1);
  }
  const size_t bytes = (size_t)p->nflat * 4;
  zl_status s = ZL_OK;
  auto dalloc = [&](void** ptr, size_t nbytes) {
    if (s) return;
    hipError_t e = hipMalloc(ptr, std::max<size_t>(nbytes, 4));
    if (e == hipSuccess) e = hipMemsetAsync(*ptr, 0, std::max<size_t>(nbytes, 4), c->stream);
    if (e != hipSuccess) s = fail(c, ZL_ERR_HIP, "zl_ppo_create: %s", hipGetErrorString(e));
  };
  dalloc((void**)&p->params, bytes);
  dalloc((void**)&p->grads, bytes);
  dalloc((void**)&p->m, bytes);
  dalloc((void**)&p->v, bytes);
  if (!s) s = p->ab.alloc(c, p->actor, mb);
  if (!s) s = p->cb.alloc(c, p->critic, mb);
  p->nb_cap = (int)std::max<long long>(std::max<long long>(cdiv(mb, kThreads), kLossMaxBlocks),
                                         zk::kHeadMaxBlocks);
  dalloc((void**)&p->gls_part, (size_t)p->nb_cap * p->A * 4);
  dalloc((void**)&p->astat_part, (size_t)p->nb_cap * 2 * 4);
  dalloc((void**)&p->vstat_part, (size_t)p->nb_cap * 4);
  // zk_kl's per-block totals, or zk_head's [A x blocks] per-component sums.
  dalloc((void**)&p->kl_part, (size_t)p->nb_cap * std::max(p->A, 1) * 4);
  // zk_reduce_all takes at least kReduceAllThreads / 64 outputs per block
  // (at most 64 split lanes).
  p->sq_cap = 1;  // + the minibatch tail's slot
  const int min_per_block = zk::kReduceAllThreads / 64;
  for (const NetLayout* nl : {&p->actor, &p->critic})
    for (int l = 0; l < nl->L; ++l)
      p->sq_cap += (int)(cdiv(cdiv((long long)nl->dims[l + 1] * nl->dims[l], 4), min_per_block) +
                         cdiv(nl->dims[l + 1], min_per_block));
  dalloc((void**)&p->sq_part, (size_t)p->sq_cap * 4);
  dalloc((void**)&p->dstate, sizeof(UpdateIn));
  if (!s) p->bptrs = (zk::BatchPtrs*)((char*)p->dstate + offsetof(UpdateIn, ptrs));
  dalloc((void**)&p->ls_old, (size_t)p->A * 4);
  dalloc((void**)&p->stat_out, 8 * 4);
  if (!s) {
    const long long pw = policy_layout(p);
    if (pw > 0) dalloc((void**)&p->polw, (size_t)pw * 4);
    if (!s) s = policy_pack(p);
  }
  if (!s && hipStreamSynchronize(c->stream) != hipSuccess)
    s = fail(c, ZL_ERR_HIP, "zl_ppo_create: stream sync failed");
  if (s) {
    zl_ppo_destroy(p);
    return s;
  }
  p->hstate = zk::DevState{};
  p->hstate.lr = 1e-3f;
  *out = p;
  return ZL_OK;
}

void zl_ppo_destroy(zl_ppo* p) {
  if (!p) return;
  if (p->c && p->c->stream) hipStreamSynchronize(p->c->stream);
  if (p->gexec) hipGraphExecDestroy(p->gexec);
  p->ab.release();
  p->cb.release();
  for (void* b : {(void*)p->params, (void*)p->grads, (void*)p->m, (void*)p->v,
                  (void*)p->gls_part, (void*)p->astat_part, (void*)p->vstat_part,
                  (void*)p->kl_part, (void*)p->sq_part, (void*)p->adv_part, (void*)p->dstate,
                  (void*)p->ls_old, (void*)p->obs_pad, (void*)p->cobs_pad, (void*)p->perm,
                  (void*)p->stat_out, (void*)p->pws, (void*)p->polw})
    if (b) hipFree(b);
  for (float* b : p->stg)
    if (b) hipFree(b);
  for (zl_ppo::ShuffleBuf& sb : p->shuf)
    if (sb.h) hipHostFree(sb.h);
  delete p;
}

zl_status zl_ppo_set_params(zl_ppo* p, const float* actor, const float* critic,
                            const float* log_std, float lr) {
  if (!p) return ZL_ERR_INVALID;
  zl_ctx* c = p->c;
  std::vector<float> host((size_t)p->nflat, 0.0f);
  ZL_HIP(c, hipMemcpyAsync(host.data(), p->params, host.size() * 4, hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  if (actor) p->actor.scatter(actor, host.data());
  if (critic) p->critic.scatter(critic, host.data());
  if (log_std) std::memcpy(host.data() + p->ls_off, log_std, (size_t)p->A * 4);
  ZL_HIP(c, hipMemcpyAsync(p->params, host.data(), host.size() * 4, hipMemcpyHostToDevice, c->stream));
  zl_status s = policy_pack(p);
  if (s) return s;
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  p->hstate.lr = lr;
  return ZL_OK;
}

zl_status zl_ppo_get_params(zl_ppo* p, float* actor, float* critic, float* log_std, float* lr) {
  if (!p) return ZL_ERR_INVALID;
  zl_ctx* c = p->c;
  std::vector<float> host((size_t)p->nflat);
  ZL_HIP(c, hipMemcpyAsync(host.data(), p->params, host.size() * 4, hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  if (actor) p->actor.gather(host.data(), actor);
  if (critic) p->critic.gather(host.data(), critic);
  if (log_std) std::memcpy(log_std, host.data() + p->ls_off, (size_t)p->A * 4);
  if (lr) *lr = p->hstate.lr;
  return ZL_OK;
}

zl_status zl_ppo_get_moments(zl_ppo* p, float* ma, float* va, float* mc, float* vc, float* mls,
                             float* vls) {
  if (!p) return ZL_ERR_INVALID;
  zl_ctx* c = p->c;
  std::vector<float> hm((size_t)p->nflat), hv((size_t)p->nflat);
  ZL_HIP(c, hipMemcpyAsync(hm.data(), p->m, hm.size() * 4, hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipMemcpyAsync(hv.data(), p->v, hv.size() * 4, hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  if (ma) p->actor.gather(hm.data(), ma);
  if (va) p->actor.gather(hv.data(), va);
  if (mc) p->critic.gather(hm.data(), mc);
  if (vc) p->critic.gather(hv.data(), vc);
  if (mls) std::memcpy(mls, hm.data() + p->ls_off, (size_t)p->A * 4);
  if (vls) std::memcpy(vls, hv.data() + p->ls_off, (size_t)p->A * 4);
  return ZL_OK;
}

zl_status zl_ppo_reset_optimizer(zl_ppo* p) {
  if (!p) return ZL_ERR_INVALID;
  zl_ctx* c = p->c;
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  ZL_HIP(c, hipMemsetAsync(p->m, 0, (size_t)p->nflat * 4, c->stream));
  ZL_HIP(c, hipMemsetAsync(p->v, 0, (size_t)p->nflat * 4, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  p->hstate.t = 0;
  p->hstate.gstep = 0;
  return ZL_OK;
}

zl_status zl_ppo_get_counters(zl_ppo* p, int* t, unsigned long long* gstep) {
  if (!p) return ZL_ERR_INVALID;
  if (t) *t = p->hstate.t;
  if (gstep) *gstep = p->hstate.gstep;
  return ZL_OK;
}

zl_status zl_ppo_update(zl_ppo* p, const zl_batch* b, const zl_ppo_config* cfg,
                        zl_ppo_stats* stats) {
  if (!p || !b || !cfg) return ZL_ERR_INVALID;
  zl_ctx* c = p->c;
  const int mode = cfg->semantics;
  if (mode != ZL_SEMANTICS_ACTOR_CRITIC && mode != ZL_SEMANTICS_GPU_TRAINER)
    return fail(c, ZL_ERR_INVALID, "zl_ppo_update: unknown semantics %d", mode);
  zl_status s = check_batch(p, b, "zl_ppo_update");
  if (s) return s;
  if (cfg->epochs < 0 || cfg->minibatches < 1 || b->n < cfg->minibatches)
    return fail(c, ZL_ERR_INVALID, "zl_ppo_update: n %lld < minibatches %d", b->n, cfg->minibatches);
  Plan pl{};
  pl.mode = mode;
  pl.n = b->n;
  pl.epochs = cfg->epochs;
  pl.mb = (int)(b->n / cfg->minibatches);  // ppo.rs:350; biped_train_gpu.rs:645
  pl.n_mb = mode == ZL_SEMANTICS_ACTOR_CRITIC ? cfg->minibatches : (int)(b->n / pl.mb);  // :1005
  if (pl.mb > p->mb_cap)
    return fail(c, ZL_ERR_INVALID, "zl_ppo_update: minibatch of %d rows > capacity %d", pl.mb,
                p->mb_cap);
  pl.shuffle = mode == ZL_SEMANTICS_ACTOR_CRITIC && cfg->shuffle;
  if ((s = plan_stage(p, b, pl.n, nullptr, 0, &pl.stage, &pl.stage_blocks, &pl.sb, &pl.share_cobs)))
    return s;
  pl.X = pl.sb.obs;
  pl.ldx = pl.sb.ld_obs;
  pl.XC = pl.sb.critic_obs;
  pl.ldxc = pl.sb.ld_critic_obs;
  if (cfg->normalize_adv) {
    size_t need = (size_t)2 * cdiv(pl.n, zl_ppo::kAdvChunk) * 4;
    if ((s = grow(p, (void**)&p->adv_part, &p->adv_part_cap, need))) return s;
  }
  if ((s = ensure_partials(p, pl.mb))) return s;
  if (pl.shuffle) {
    size_t cap = p->perm_cap * 4;
    if ((s = grow(p, (void**)&p->perm, &cap, (size_t)pl.epochs * pl.n * 4 + 4))) return s;
    p->perm_cap = cap / 4;
    zl_ppo::ShuffleBuf& sb = p->shuf[p->shuf_cur];
    if (!(sb.n == pl.n && sb.epochs == pl.epochs && sb.minibatches == cfg->minibatches &&
          sb.t == p->hstate.t)) {
      hipError_t e = shuffle_orders(sb, pl.n, pl.epochs, cfg->minibatches, p->hstate.t);
      if (e != hipSuccess)
        return fail(c, ZL_ERR_HIP, "zl_ppo_update: hipHostMalloc (shuffle orders): %s",
                    hipGetErrorString(e));
    }
  }
  zk::PpoParams& pp = pl.pp;
  pp.mode = mode;
  pp.A = p->A;
  pp.mb = pl.mb;
  pp.n_mb = pl.n_mb;
  pp.clip = cfg->clip;
  pp.entropy_coef = cfg->entropy_coef;
  pp.value_coef = cfg->value_coef;
  pp.scale = 1.0f / (float)pl.mb;
  pp.max_grad_norm = cfg->max_grad_norm;
  pp.desired_kl = cfg->desired_kl;
  pp.lr_min = cfg->lr_min;
  pp.lr_max = cfg->lr_max;
  pp.adaptive_lr = cfg->adaptive_lr;
  pp.early_stop = mode == ZL_SEMANTICS_GPU_TRAINER ? cfg->early_stop : 0;
  pp.clamp_ls = mode == ZL_SEMANTICS_ACTOR_CRITIC && cfg->clamp_log_std ? 1 : 0;
  pp.beta1 = 0.9f;
  pp.beta2 = 0.999f;
  pp.eps = 1e-8f;

  // The launch sequence depends only on these: shapes, strides, layouts, the
  // configuration and the generation of the handle's buffers. The caller's
  // pointers reach the graph through p->bptrs, the per-update scalars through
  // p->dstate.
  char key[512];
  snprintf(key, sizeof(key),
           "%d|%lld|%d|%d|%d|%d|%d|%d|%d|%u|%d|%d|%d|%a|%a|%a|%a|%a|%a|%a|%d|%d|%d|%d|%d|%llu",
           mode, pl.n, pl.mb, pl.n_mb, pl.epochs, b->ld_obs, b->ld_critic_obs, b->ld_action,
           b->ld_mean_old, b->feature_major, (int)pl.share_cobs, (int)(b->mean_old != nullptr),
           (int)pl.shuffle, (double)cfg->clip, (double)cfg->entropy_coef, (double)cfg->value_coef,
           (double)cfg->max_grad_norm, (double)cfg->desired_kl, (double)cfg->lr_min,
           (double)cfg->lr_max, cfg->adaptive_lr, cfg->early_stop, cfg->normalize_adv,
           cfg->clamp_log_std, cfg->shuffle, p->gen);
  const bool eager = c->timing_kernel != -1;
  if (!eager && (!p->gexec || p->gkey != key)) {
    const auto t0 = std::chrono::steady_clock::now();
    if (p->gexec) {
      hipGraphExecDestroy(p->gexec);
      p->gexec = nullptr;
    }
    p->gkey.clear();
    ZL_HIP(c, hipStreamSynchronize(c->stream));
    ZL_HIP(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    s = enqueue_update(p, cfg, pl);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &graph);
    if (s) {
      if (graph) hipGraphDestroy(graph);
      return s;
    }
    if (e != hipSuccess)
      return fail(c, ZL_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(&p->gexec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (e != hipSuccess) {
      p->gexec = nullptr;
      return fail(c, ZL_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    p->gkey = key;
    p->captures += 1;
    p->capture_ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }
  // Per-update device scalars: persistent lr / t / gstep, everything else
  // reset; the caller's batch pointers beside them.
  UpdateIn in{};
  zk::DevState& st = in.st;
  st = p->hstate;
  st.active = 1;
  st.epochs_run = 0;
  st.mb_in_epoch = 0;
  st.ep_kl = st.ep_surr = st.ep_vloss = st.ep_ent = 0.f;
  for (float& x : st.stats) x = 0.f;
  st.stats[4] = st.lr;
  st.scale[0] = st.scale[1] = st.scale[2] = 1.f;
  st.norm[0] = st.norm[1] = st.norm[2] = 0.f;
  st.last_kl = 0.f;
  if (mode == ZL_SEMANTICS_ACTOR_CRITIC) {
    st.bc1 = 1.f;
    st.bc2 = 1.f;
  }
  in.ptrs = batch_ptrs(b);
  ZL_HIP(c, hipMemcpyAsync(p->dstate, &in, sizeof(in), hipMemcpyHostToDevice, c->stream));
  ZL_HIP(c, hipMemcpyAsync(p->ls_old, p->params + p->ls_off, (size_t)p->A * 4,
                           hipMemcpyDeviceToDevice, c->stream));
  if (pl.shuffle)
    ZL_HIP(c, hipMemcpyAsync(p->perm, p->shuf[p->shuf_cur].h, (size_t)pl.epochs * pl.n * 4,
                             hipMemcpyHostToDevice, c->stream));
  if (eager) {
    if ((s = enqueue_update(p, cfg, pl))) return s;
  } else {
    ZL_HIP(c, hipGraphLaunch(p->gexec, c->stream));
  }
  if (pl.shuffle) {
    // The next update's orders while the device runs this one (every
    // minibatch of every epoch takes one Adam step under these semantics).
    // The other buffer's last upload finished with the previous call.
    p->shuf_cur ^= 1;
    zl_ppo::ShuffleBuf& nb = p->shuf[p->shuf_cur];
    // On an allocation failure the buffer's key stays unset and the next
    // call computes its orders itself.
    (void)shuffle_orders(nb, pl.n, pl.epochs, cfg->minibatches,
                         p->hstate.t + pl.epochs * cfg->minibatches);
  }
  ZL_HIP(c, hipMemcpyAsync(&st, p->dstate, sizeof(st), hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  p->hstate.lr = st.lr;
  p->hstate.t = st.t;
  p->hstate.gstep = st.gstep;
  if (stats) {
    stats->kl = st.stats[0];
    stats->surrogate = st.stats[1];
    stats->value_loss = st.stats[2];
    stats->entropy = st.stats[3];
    stats->lr = st.stats[4];
    stats->epochs_run = st.epochs_run;
    stats->last_kl = st.last_kl;
    stats->grad_norm[0] = st.norm[0];
    stats->grad_norm[1] = st.norm[1];
    stats->grad_norm[2] = st.norm[2];
  }
  return ZL_OK;
}

zl_status zl_ppo_graph_info(zl_ppo* p, long long* captures, double* last_capture_ms) {
  if (!p) return ZL_ERR_INVALID;
  if (captures) *captures = p->captures;
  if (last_capture_ms) *last_capture_ms = p->capture_ms;
  return ZL_OK;
}

zl_status zl_ppo_get_grads(zl_ppo* p, float* actor, float* critic, float* log_std) {
  if (!p) return ZL_ERR_INVALID;
  zl_ctx* c = p->c;
  std::vector<float> host((size_t)p->nflat);
  ZL_HIP(c, hipMemcpyAsync(host.data(), p->grads, host.size() * 4, hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  if (actor) p->actor.gather(host.data(), actor);
  if (critic) p->critic.gather(host.data(), critic);
  if (log_std) std::memcpy(log_std, host.data() + p->ls_off, (size_t)p->A * 4);
  return ZL_OK;
}

zl_status zl_ppo_minibatch_grads(zl_ppo* p, const zl_batch* b, const zl_ppo_config* cfg,
                                 long long row0, int rows, const int* perm_dev, float* stats) {
  if (!p || !b || !cfg) return ZL_ERR_INVALID;
  zl_ctx* c = p->c;
  zl_status s = check_batch(p, b, "zl_ppo_minibatch_grads");
  if (s) return s;
  if (rows < 1 || rows > p->mb_cap || row0 < 0 || row0 + rows > b->n)
    return fail(c, ZL_ERR_INVALID, "zl_ppo_minibatch_grads: rows [%lld, %lld) outside [0, %lld) or "
                "more than %d", row0, row0 + rows, b->n, p->mb_cap);
  // The minibatch's samples are staged as rows 0 .. rows-1 (gathered through
  // perm_dev when given), batch-major and aligned for the layer-0 GEMMs.
  Plan pl{};
  if ((s = plan_stage(p, b, rows, perm_dev, row0, &pl.stage, &pl.stage_blocks, &pl.sb,
                      &pl.share_cobs)))
    return s;
  const zk::BatchPtrs hp = batch_ptrs(b);
  ZL_HIP(c, hipMemcpyAsync(p->bptrs, &hp, sizeof(hp), hipMemcpyHostToDevice, c->stream));
  if ((s = launch(c, K_STAGE, (unsigned)pl.stage_blocks, 1, 1, pl.stage))) return s;
  const int A = p->A;
  if ((s = ensure_partials(p, rows))) return s;
  const NetView v[2] = {{&p->actor, &p->ab, pl.sb.obs, pl.sb.ld_obs, pl.sb.ld_obs},
                        {&p->critic, &p->cb, pl.sb.critic_obs, pl.sb.ld_critic_obs,
                         pl.sb.ld_critic_obs}};
  PassCounts pc;
  if ((s = minibatch_pass(p, v, nullptr, nullptr, 0, rows, &pl.sb, cfg, 1.0f / (float)rows,
                          nullptr, &pc)))
    return s;
  // Fixed-order sums of the per-block partials.
  auto reduce = [&](const float* part, int width, int parts, float* out) {
    zk::SplitReduceArgs r{};
    r.part = part;
    r.out = out;
    r.mn = width;
    r.cols = width;
    r.ldo = width;
    r.splits = parts;
    return launch_splitk_reduce(c, r);
  };
  if ((s = reduce_rows(c, p->gls_part, A, pc.nb_a, p->grads + p->ls_off))) return s;
  if ((s = reduce_rows(c, p->astat_part, 2, pc.nb_a, p->stat_out))) return s;
  if ((s = reduce(p->vstat_part, 1, pc.nb_v, p->stat_out + 2))) return s;
  float h[3];
  ZL_HIP(c, hipMemcpyAsync(h, p->stat_out, sizeof(h), hipMemcpyDeviceToHost, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  if (stats) {
    stats[0] = h[0];  // surrogate
    stats[1] = h[2];  // value loss
    stats[2] = h[1];  // kl
  }
  return ZL_OK;
}

static void policy_net(zk::PolicyNet& q, const zl_ppo* p, int net, const float* x, int ldx,
                       const float* norm, float* out, int ldo) {
  const NetLayout& nl = net ? p->critic : p->actor;
  q = zk::PolicyNet{};
  q.wp = p->polw;
  q.x = x;
  q.ldx = ldx;
  q.norm = norm;
  q.out = out;
  q.ldo = ldo;
  q.L = nl.L;
  for (int l = 0; l <= nl.L; ++l) q.dims[l] = nl.dims[l];
  for (int l = 0; l < nl.L; ++l) {
    q.wp_off[l] = p->polw_off[net][l];
    q.b_off[l] = nl.b_off[l];
  }
}

static zl_status chunked_forward(zl_ppo* p, bool critic, const float* x, int ld, long long n,
                                 float* out, int ld_out, int cols) {
  zl_ctx* c = p->c;
  const NetLayout& nl = critic ? p->critic : p->actor;
  const NetBuffers& nb = critic ? p->cb : p->ab;
  if (!x || !out || n < 0 || ld < nl.dims[0] || ld_out < cols)
    return fail(c, ZL_ERR_INVALID, "forward: bad argument");
  if (n > 0 && n <= kPolicyFusedRows && c->fused_policy && p->polw_net[critic ? 1 : 0]) {
    zk::PolicyArgs a{};
    policy_net(a.net[0], p, critic ? 1 : 0, x, ld, nullptr, out, ld_out);
    a.params = p->params;
    a.rows = n;
    return launch(c, K_POLICY, (unsigned)cdiv(n, zk::kPolicyRows), 1, 1, a, 0, zk::kPolicyThreads);
  }
  // The output layer writes straight into the caller's rows.
  auto desc = [&](const NetBuffers& b, const float* xx, int rows, long long r0, int l) {
    GemmDesc d = fwd_desc(nl, b, p->params, xx, ld, nullptr, rows, nullptr, l);
    if (l == nl.L - 1) {
      d.C = out + (size_t)r0 * ld_out;
      d.ldc = ld_out;
    }
    return d;
  };
  // The other net's activation buffers can hold a second chunk when every
  // layer of this net fits their widths (the critic's in the actor's, same
  // hidden widths): two chunks then run as one grouped launch per layer.
  const NetLayout& onl = critic ? p->actor : p->critic;
  const NetBuffers& onb = critic ? p->ab : p->cb;
  bool borrow = onl.L == nl.L;
  for (int l = 1; borrow && l < nl.L; ++l) borrow = onb.ld[l] >= nl.dims[l];
  long long r0 = 0;
  if (borrow) {
    for (; r0 + p->mb_cap < n; r0 += 2LL * p->mb_cap) {
      const int rows0 = p->mb_cap;
      const int rows1 = (int)std::min<long long>(p->mb_cap, n - r0 - rows0);
      const float* x0 = x + (size_t)r0 * ld;
      const float* x1 = x + (size_t)(r0 + rows0) * ld;
      for (int l = 0; l < nl.L; ++l) {
        GemmDesc d[2] = {desc(nb, x0, rows0, r0, l), desc(onb, x1, rows1, r0 + rows0, l)};
        zl_status s = run_gemm_batch(c, d, 2);
        if (s) return s;
      }
    }
  }
  for (; r0 < n; r0 += p->mb_cap) {
    const int rows = (int)std::min<long long>(p->mb_cap, n - r0);
    for (int l = 0; l < nl.L; ++l) {
      GemmDesc d = desc(nb, x + (size_t)r0 * ld, rows, r0, l);
      zl_status s = run_gemm_batch(c, &d, 1);
      if (s) return s;
    }
  }
  return ZL_OK;
}

zl_status zl_ppo_act(zl_ppo* p, const float* obs_norm, const float* obs, int ld_obs,
                     const float* critic_norm, const float* cobs, int ld_cobs, long long n,
                     const float* eps, float* action, float* logp, float* mean, int ld_mean,
                     float* value) {
  if (!p) return ZL_ERR_INVALID;
  zl_ctx* c = p->c;
  const int od = p->actor.dims[0], cd = p->critic.dims[0], A = p->A;
  if (n < 0 || !obs || !eps || !action || !logp || ld_obs < od || (mean && ld_mean < A) ||
      (value && (!cobs || ld_cobs < cd)) || (!value && critic_norm))
    return fail(c, ZL_ERR_INVALID, "zl_ppo_act: bad argument");
  if (n == 0) return ZL_OK;
  if (n <= kPolicyFusedRows && c->fused_policy && A <= 32 && p->polw_net[0] &&
      (!value || p->polw_net[1])) {
    // One launch: normalise, both nets' layers, sampling (zk_policy).
    zk::PolicyArgs a{};
    policy_net(a.net[0], p, 0, obs, ld_obs, obs_norm, mean, ld_mean);
    if (value) policy_net(a.net[1], p, 1, cobs, ld_cobs, critic_norm, value, 1);
    a.params = p->params;
    a.log_std = p->params + p->ls_off;
    a.eps = eps;
    a.lde = A;
    a.action = action;
    a.lda = A;
    a.logp = logp;
    a.rows = n;
    a.A = A;
    a.sample = 1;
    return launch(c, K_POLICY, (unsigned)cdiv(n, zk::kPolicyRows), value ? 2 : 1, 1, a, 0,
                  zk::kPolicyThreads);
  }
  // Normalised inputs go to the padded staging buffers (16-byte aligned rows
  // for the layer-0 GEMM); raw inputs that are already normalised are read
  // in place.
  const int odp = (int)round_up(od, 4), cdp = (int)round_up(cd, 4);
  const int chunk = (int)std::min<long long>(p->mb_cap, n);
  zl_status s = ZL_OK;
  if (obs_norm) {
    size_t cap = p->obs_pad_floats * 4;
    if ((s = grow(p, (void**)&p->obs_pad, &cap, (size_t)chunk * odp * 4))) return s;
    p->obs_pad_floats = cap / 4;
  }
  if (critic_norm) {
    size_t cap = p->cobs_pad_floats * 4;
    if ((s = grow(p, (void**)&p->cobs_pad, &cap, (size_t)chunk * cdp * 4))) return s;
    p->cobs_pad_floats = cap / 4;
  }
  const int La = p->actor.L, Lc = p->critic.L;
  for (long long r0 = 0; r0 < n; r0 += chunk) {
    const int rows = (int)std::min<long long>(chunk, n - r0);
    NetView v[2] = {{&p->actor, &p->ab, obs + (size_t)r0 * ld_obs, ld_obs},
                    {&p->critic, &p->cb, value ? cobs + (size_t)r0 * ld_cobs : nullptr, ld_cobs}};
    if (obs_norm) {
      if ((s = zl_norm_normalize(c, obs_norm, od, v[0].x, ld_obs, rows, p->obs_pad, odp))) return s;
      v[0].x = p->obs_pad;
      v[0].ldx = odp;
    }
    if (critic_norm) {
      if ((s = zl_norm_normalize(c, critic_norm, cd, v[1].x, ld_cobs, rows, p->cobs_pad, cdp)))
        return s;
      v[1].x = p->cobs_pad;
      v[1].ldx = cdp;
    }
    s = value ? pair_forward(c, v, p->params, nullptr, rows, nullptr)
              : net_forward(c, p->actor, p->ab, p->params, v[0].x, v[0].ldx, nullptr, rows, nullptr);
    if (s) return s;
    zk::SampleArgs sa{};
    sa.mean = p->ab.act[La];
    sa.ldm = p->ab.ld[La];
    sa.log_std = p->params + p->ls_off;
    sa.eps = eps + (size_t)r0 * A;
    sa.action = action + (size_t)r0 * A;
    sa.logp = logp + r0;
    sa.rows = rows;
    sa.A = A;
    sa.lde = A;
    sa.lda = A;
    if ((s = launch_sample(c, sa))) return s;
    if (mean && (s = copy_rows(c, mean + (size_t)r0 * ld_mean, ld_mean, p->ab.act[La], p->ab.ld[La],
                               A, rows, nullptr, 0, nullptr, false)))
      return s;
    if (value && (s = copy_rows(c, value + r0, 1, p->cb.act[Lc], p->cb.ld[Lc], 1, rows, nullptr, 0,
                                nullptr, false)))
      return s;
  }
  return ZL_OK;
}

zl_status zl_ppo_values(zl_ppo* p, const float* cobs, int ld, long long n, float* values) {
  if (!p) return ZL_ERR_INVALID;
  return chunked_forward(p, true, cobs, ld, n, values, 1, 1);
}

zl_status zl_ppo_actor_mean(zl_ppo* p, const float* obs, int ld, long long n, float* mean,
                            int ld_mean) {
  if (!p) return ZL_ERR_INVALID;
  return chunked_forward(p, false, obs, ld, n, mean, ld_mean, p->A);
}

}  // extern "C"

// ---- accessors for the checkpoint code (checkpoint.cpp)
namespace zl {

zl_ctx* ppo_ctx(zl_ppo* p) { return p->c; }

void ppo_dims(const zl_ppo* p, std::vector<int>* actor, std::vector<int>* critic) {
  *actor = p->actor.dims;
  *critic = p->critic.dims;
}

zl_status ppo_set_moments(zl_ppo* p, const float* ma, const float* va, const float* mc,
                          const float* vc, const float* mls, const float* vls) {
  zl_ctx* c = p->c;
  std::vector<float> hm((size_t)p->nflat, 0.0f), hv((size_t)p->nflat, 0.0f);
  p->actor.scatter(ma, hm.data());
  p->actor.scatter(va, hv.data());
  p->critic.scatter(mc, hm.data());
  p->critic.scatter(vc, hv.data());
  std::memcpy(hm.data() + p->ls_off, mls, (size_t)p->A * 4);
  std::memcpy(hv.data() + p->ls_off, vls, (size_t)p->A * 4);
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  ZL_HIP(c, hipMemcpyAsync(p->m, hm.data(), hm.size() * 4, hipMemcpyHostToDevice, c->stream));
  ZL_HIP(c, hipMemcpyAsync(p->v, hv.data(), hv.size() * 4, hipMemcpyHostToDevice, c->stream));
  ZL_HIP(c, hipStreamSynchronize(c->stream));
  return ZL_OK;
}

void ppo_set_counters(zl_ppo* p, int t, unsigned long long gstep) {
  p->hstate.t = t;
  p->hstate.gstep = gstep;
}

}  // namespace zl
