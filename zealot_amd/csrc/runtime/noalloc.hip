// noalloc.hip — the allocation-free variant of zl_grad_clip_scale.
//
// Its per-block sum-of-squares partials live in a file-scope device array of
// fixed size instead of the context's growable scratch, so the call makes no
// hipMalloc / hipFree and can be issued under HIP graph capture or from a loop
// that must not allocate. The array is one per GPU (each device holds its own
// copy while the process runs, 256 KiB); its device address is looked up with
// hipGetSymbolAddress when a context is created on the device (kept once a
// lookup succeeds) and only that address is handed to kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.hpp"

namespace {

// Partials of one call: one float per 2048-element chunk of each tensor
// (at least one per tensor), so up to ~33.5 M gradient elements. The array
// holds kSlots such regions; every context claims one at zl_init and gives
// it back at zl_destroy, so calls of different contexts never share
// partials, and the calls of one context are ordered on its one stream.
constexpr int kSlotFloats = 16384;
constexpr int kSlots = 4;
constexpr int kChunk = 2048;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kSlots * kSlotFloats];

std::mutex g_mu;
float* g_ptr[kMaxDevices] = {};      // set only by a successful lookup
unsigned g_used[kMaxDevices] = {};   // claimed slots, one bit each

}  // namespace

namespace zl {

// Called by zl_init with `device` current: looks up the device address of
// `scratch` on that device (until a lookup succeeds) and claims a free slot.
void noalloc_setup(zl_ctx* c) {
  std::lock_guard<std::mutex> lock(g_mu);
  const int d = c->device;
  c->noalloc_scratch = nullptr;
  c->noalloc_slot = -1;
  c->noalloc_err = hipSuccess;
  if (d < 0 || d >= kMaxDevices) {
    c->noalloc_err = hipErrorInvalidDevice;
    return;
  }
  if (!g_ptr[d]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      c->noalloc_err = e != hipSuccess ? e : hipErrorInvalidSymbol;
      return;
    }
    g_ptr[d] = (float*)p;
  }
  for (int s = 0; s < kSlots; ++s)
    if (!(g_used[d] & (1u << s))) {
      g_used[d] |= 1u << s;
      c->noalloc_slot = s;
      c->noalloc_scratch = g_ptr[d] + (size_t)s * kSlotFloats;
      return;
    }
}

// Called by zl_destroy after the context's stream has drained.
void noalloc_release(zl_ctx* c) {
  std::lock_guard<std::mutex> lock(g_mu);
  const int d = c->device;
  if (c->noalloc_slot >= 0 && d >= 0 && d < kMaxDevices) g_used[d] &= ~(1u << c->noalloc_slot);
  c->noalloc_slot = -1;
  c->noalloc_scratch = nullptr;
}

}  // namespace zl

using namespace zl;

extern "C" zl_status zl_grad_clip_scale_noalloc(zl_ctx* c, const zl_tensor* tensors, int count,
                                                float max_norm, float* scale_dev, float* norm_dev) {
  if (!c) return ZL_ERR_INVALID;
  if (!c->noalloc_scratch) {
    if (c->noalloc_err != hipSuccess)
      return fail(c, ZL_ERR_HIP, "zl_grad_clip_scale_noalloc: device scratch unavailable (%s)",
                  hipGetErrorString(c->noalloc_err));
    return fail(c, ZL_ERR_INVALID,
                "zl_grad_clip_scale_noalloc: all %d static scratch slots of this GPU are held by "
                "other contexts", kSlots);
  }
  if (!tensors || !scale_dev || count < 1 || count > zk::kMaxNormTensors)
    return fail(c, ZL_ERR_INVALID, "zl_grad_clip_scale_noalloc: bad argument (count %d)", count);
  zk::SumsqMultiArgs a{};
  long long blk = 0;
  for (int j = 0; j < count; ++j) {
    if (!tensors[j].ptr && tensors[j].n)
      return fail(c, ZL_ERR_INVALID, "zl_grad_clip_scale_noalloc: tensor %d is NULL", j);
    a.x[j] = tensors[j].ptr;
    a.n[j] = (long long)tensors[j].n;
    a.blk0[j] = (int)std::min<long long>(blk, kSlotFloats + 1);
    blk += std::max<long long>(1, cdiv((long long)tensors[j].n, kChunk));
  }
  if (blk > kSlotFloats)
    return fail(c, ZL_ERR_INVALID,
                "zl_grad_clip_scale_noalloc: %lld partials needed, the static scratch holds %d "
                "(at most about %d gradient elements per call)",
                blk, kSlotFloats, kSlotFloats * kChunk);
  a.blk0[count] = (int)blk;
  a.count = count;
  a.chunk = kChunk;
  a.part = c->noalloc_scratch;
  zl_status s = launch(c, K_SUMSQ_MULTI, (unsigned)blk, 1, 1, a);
  if (s) return s;
  zk::ClipScaleArgs cs{};
  cs.part = c->noalloc_scratch;
  cs.nparts = (int)blk;
  cs.max_norm = max_norm;
  cs.scale = scale_dev;
  cs.norm = norm_dev;
  return launch(c, K_CLIP_SCALE, 1, 1, 1, cs, 0, 64);
}
