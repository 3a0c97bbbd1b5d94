// Shared device-side definitions for the Synaptik HIP backend (gfx950 / CDNA4).
//
// Numerical conventions follow the reference CPU backend's scalar oracles:
//   * activations are evaluated in binary64 and narrowed once to binary32
//     (modules/backend/cpu/.../reference/CpuScalarReferenceKernel.java:1213-1217,1736-1737);
//   * RELU is Math.max(x, +0.0): NaN propagates and -0.0 becomes +0.0;
//   * activation gradients are computed from the activation OUTPUT y with the exact
//     operation order of modules/compiler/.../ElementwiseGradientRules.java:205-210.
// All HIP sources are compiled with -ffp-contract=off so that elementwise kernels perform
// the same rounded operations as the oracle (no silent FMA contraction).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kernels.h"

namespace shk {

typedef float floatx16 __attribute__((ext_vector_type(16)));

enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_TANH = 2, ACT_SIGMOID = 3 };



__device__ __forceinline__ bool is_finite(float x) {
  return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u;
}
__device__ __forceinline__ bool is_finite(double x) {
  return (__double_as_longlong(x) & 0x7ff0000000000000ll) != 0x7ff0000000000000ll;
}

// Math.max(x, +0.0) narrowed: NaN stays NaN, -0.0 and negatives become +0.0.
__device__ __forceinline__ float relu_f(float x) {
  return (x > 0.0f || x != x) ? x : 0.0f;
}

// Stable two-branch logistic in binary64 (CpuScalarReferenceKernel.java:1213-1217).
__device__ __forceinline__ float sigmoid_f(float xf) {
  double x = (double)xf;
  double r;
  if (x >= 0.0) {
    r = 1.0 / (1.0 + exp(-x));
  } else {
    double e = exp(x);
    r = e / (1.0 + e);
  }
  return (float)r;
}

__device__ __forceinline__ float tanh_f(float x) { return (float)tanh((double)x); }

__device__ __forceinline__ float apply_act(int act, float z) {
  switch (act) {
    case ACT_RELU: return relu_f(z);
    case ACT_TANH: return tanh_f(z);
    case ACT_SIGMOID: return sigmoid_f(z);
    default: return z;
  }
}

// Cotangent of the activation input from the upstream cotangent g and activation output y.
//   RELU:    WHERE(x > 0, g, 0)   (x > 0 exactly when y > 0)
//   TANH:    g * (1 - y*y)
//   SIGMOID: (g * y) * (1 - y)
__device__ __forceinline__ float act_grad(int act, float g, float y) {
  switch (act) {
    case ACT_RELU: return y > 0.0f ? g : 0.0f;
    case ACT_TANH: { float yy = y * y; float d = 1.0f - yy; return g * d; }
    case ACT_SIGMOID: { float gy = g * y; float d = 1.0f - y; return gy * d; }
    default: return g;
  }
}

// Java Math.max semantics on binary32: NaN wins, +0.0 beats -0.0.
__device__ __forceinline__ float java_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == 0.0f && b == 0.0f) return __uint_as_float(__float_as_uint(a) & __float_as_uint(b));
  return a > b ? a : b;
}

// Streaming (non-temporal) 16-byte loads and stores for data touched once per kernel: they do
// not displace cache lines other work still needs, which lifts the large row kernels' HBM rate.
typedef float float4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream(const float4* a) {
  const float4v t = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(a));
  return make_float4(t[0], t[1], t[2], t[3]);
}
__device__ __forceinline__ void st_stream(float4* a, float4 v) {
  __builtin_nontemporal_store(float4v{v.x, v.y, v.z, v.w}, reinterpret_cast<float4v*>(a));
}

// Wave64 reductions through cross-lane shuffles (DPP/permute on CDNA).
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = java_max(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
  return v;
}

// Block-wide reductions: wave shuffle tree, then an LDS tree over the waves.
template <int NT>
__device__ __forceinline__ double block_sum(double v, double* lds) {
  constexpr int NW = NT / 64;
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (NW == 1) return v;
  __syncthreads();
  if (l == 0) lds[w] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int i = 0; i < NW; ++i) r += lds[i];
  return r;
}
template <int NT>
__device__ __forceinline__ float block_max(float v, float* lds) {
  constexpr int NW = NT / 64;
  v = wave_max(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (NW == 1) return v;
  __syncthreads();
  if (l == 0) lds[w] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = java_max(r, lds[i]);
  return r;
}

// MEAN of the per-row losses: binary64 partials of rows 4i .. 4i+3 (((l0 + l1) + l2) + l3),
// summed over i in a 256-strided order and a block tree, then (float)sum / (float)R.
__device__ __forceinline__ void ce_mean_block(const float* __restrict__ row_loss, int64_t R,
                                              float* loss, double* dl) {
  const int64_t P = (R + 3) / 4;
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < P; i += 256) {
    double q[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) q[w] = 4 * i + w < R ? (double)row_loss[4 * i + w] : 0.0;
    s += ((q[0] + q[1]) + q[2]) + q[3];
  }
  s = block_sum<256>(s, dl);
  if (threadIdx.x == 0) loss[0] = (float)s / (float)(double)R;
}

}  // namespace shk
