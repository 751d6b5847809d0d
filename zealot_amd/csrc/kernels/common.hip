// common.hip — shared device helpers for the gfx950 code object.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "zk_args.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace zk {

constexpr int kThreads = 256;
constexpr float kLogSqrt2Pi = 0.9189385f;  // zealot-rl/src/ppo.rs:18

// zealot-rl/src/net.rs:14-16: x > 0 ? x : exp(x) - 1 (not expm1). Used in
// the GEMM epilogues over every hidden activation, so exp is the hardware
// exp2 (v_exp_f32) of x * log2(e): on the negative branch the result lies in
// (-1, 0] with an absolute error below ~2e-7 (rounding the product x * log2(e)
// costs exp(x) * |x| * 2^-24 <= 2^-24 / e, plus about one ulp of exp2).
__device__ __forceinline__ float elu(float x) { return x > 0.0f ? x : __expf(x) - 1.0f; }

// zealot-rl/src/net.rs:21-23: derivative from the post-activation.
__device__ __forceinline__ float elu_grad_from_act(float a) { return a > 0.0f ? 1.0f : a + 1.0f; }

__device__ __forceinline__ float clampf(float x, float lo, float hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// Rust f32::powi lowering (__powisf2): square-and-multiply from the low bit,
// plain f32 multiplies. Bit-identical to the host computation.
__device__ __forceinline__ float powi_f32(float x, int n) {
  unsigned int k = n < 0 ? -(unsigned int)n : (unsigned int)n;
  float y = (k & 1u) ? x : 1.0f;
  while (k >>= 1) {
    x = x * x;
    if (k & 1u) y = y * x;
  }
  return n < 0 ? 1.0f / y : y;
}

// Deterministic butterfly sum over the 64 lanes of a wavefront (lane 0's
// result is the same on every run; all lanes hold a total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = v + __shfl_xor(v, m, 64);
  return v;
}

// Fixed-order sum of x[0], x[stride], ... (n terms) by one wavefront: lane l
// adds terms l, l+64, ... in order, then the lanes are combined by wave_sum.
// Loads are issued 8 at a time ahead of their adds (latency, not bandwidth,
// bounds these short reductions).
__device__ __forceinline__ float wave_sum_strided(const float* x, int n, int stride) {
  const int lane = threadIdx.x & 63;
  float s = 0.f;
  for (int i0 = lane; i0 < n; i0 += 8 * 64) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * 64;
      t[u] = i < n ? x[(long long)i * stride] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (i0 + u * 64 < n) s += t[u];
  }
  return wave_sum(s);
}

// Deterministic in-block tree sum over N values held one per thread (N =
// the block size). `sm` must hold N floats. Returns the total in every thread.
template <int N = kThreads>
__device__ __forceinline__ float block_sum(float v, float* sm) {
  const int t = threadIdx.x;
  sm[t] = v;
  __syncthreads();
#pragma unroll
  for (int s = N / 2; s > 0; s >>= 1) {
    if (t < s) sm[t] = sm[t] + sm[t + s];
    __syncthreads();
  }
  float r = sm[0];
  __syncthreads();
  return r;
}

}  // namespace zk
