// Row softmax / log-softmax / log-sum-exp and the MSE and index categorical cross-entropy losses.
//
// Softmax follows CpuSoftmaxReferenceKernel.evaluateFloat (reference/CpuSoftmaxReferenceKernel.java:104-146):
//   maximum by Math.max; a +inf maximum maps +inf entries to NaN and the rest to 0 (softmax) or
//   -inf (log-softmax); a row containing -inf (and no NaN) is evaluated unshifted (shift 0);
//   addends are (float)exp((double)(x - shift)); the result is (float)exp(shift)/sum or
//   shift - (float)log(sum). The GPU forms the addends with exp_f32 (fexp.h), which returns
//   that binary32 value or one of its neighbours (at most 1 ulp away; 0.46% of arguments), and
//   rows held in registers multiply by a once-rounded reciprocal of the sum.
//   The reference sums addends with Kahan compensation in binary32 (error within about
//   2 ulp of the exact sum). Register-held rows sum each lane's 4V binary32 addends pairwise in
//   binary32 (positive addends: error within log2(4V) ulp), combine the lanes in binary64
//   through a fixed tree and round once; streamed rows sum in binary64 throughout. Both sums are
//   within a few binary32 ulps of the exact sum (reduction-order difference).
// One 256-thread workgroup owns one row; rows up to 4096 wide are held in registers
// (one HBM read and one write per element), wider rows are streamed three times.
#include "common.h"
#include "fexp.h"
#include "kernels.h"
#include <algorithm>

namespace shk {
namespace {

constexpr int SM_NT = 256;

__device__ __forceinline__ int block_or(int v, int* lds) {
  v = wave_or(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = 0;
#pragma unroll
  for (int i = 0; i < SM_NT / 64; ++i) r |= lds[i];
  return r;
}

struct RowStats {
  float shift;
  float sum;
  bool pos_inf;
};

__device__ __forceinline__ float shifted_exp(float x, float shift) {
  return exp_f32(x - shift);
}

// V float4 per thread in registers (C <= V * 4 * SM_NT, C % 4 == 0).
//
// The row statistics use the hardware max / min (v_max_f32 / v_min_f32, which skip NaN and need
// not order signed zeros) and restore Math.max semantics where they differ, in a branch taken
// only by rows whose maximum is +inf or a zero: a NaN anywhere makes the maximum NaN, and a zero
// maximum is +0 when any element is +0. A row holds -inf exactly when its minimum is -inf.
// A row with a NaN and no +inf already gives NaN everywhere through the sum, as the reference's
// NaN shift does.
template <int V>
__global__ void __launch_bounds__(SM_NT) softmax_fwd_regs(const float* __restrict__ x,
                                                          float* __restrict__ y, float* lse,
                                                          int64_t C, int log_softmax) {
  __shared__ double dl[SM_NT / 64];
  __shared__ float fmx[SM_NT / 64], fmn[SM_NT / 64];
  __shared__ int il[SM_NT / 64], il2[SM_NT / 64];
  const int64_t r = blockIdx.x;
  const float4* xr = reinterpret_cast<const float4*>(x + r * C);
  float4* yr = reinterpret_cast<float4*>(y + r * C);
  const int C4 = (int)(C / 4);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float4 v[V];
  float m = -INFINITY, mn = INFINITY;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + i * SM_NT;
    if (c < C4) {
      v[i] = ld_stream(&xr[c]);
      m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
      mn = fminf(mn, fminf(fminf(v[i].x, v[i].y), fminf(v[i].z, v[i].w)));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    m = fmaxf(m, __shfl_xor(m, o, 64));
    mn = fminf(mn, __shfl_xor(mn, o, 64));
  }
  if (lane == 0) { fmx[w] = m; fmn[w] = mn; }
  __syncthreads();
  m = fmx[0];
  mn = fmn[0];
#pragma unroll
  for (int i = 1; i < SM_NT / 64; ++i) {
    m = fmaxf(m, fmx[i]);
    mn = fminf(mn, fmn[i]);
  }
  if (m == INFINITY || m == 0.0f) {  // block-uniform, rare
    int nan = 0, pos_zero = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int c = threadIdx.x + i * SM_NT;
      if (c < C4) {
        nan |= (v[i].x != v[i].x) | (v[i].y != v[i].y) | (v[i].z != v[i].z) | (v[i].w != v[i].w);
        pos_zero |= (__float_as_uint(v[i].x) == 0u) | (__float_as_uint(v[i].y) == 0u) |
                    (__float_as_uint(v[i].z) == 0u) | (__float_as_uint(v[i].w) == 0u);
      }
    }
    nan = wave_or(nan);
    pos_zero = wave_or(pos_zero);
    if (lane == 0) { il[w] = nan; il2[w] = pos_zero; }
    __syncthreads();
    nan = 0;
    pos_zero = 0;
#pragma unroll
    for (int i = 0; i < SM_NT / 64; ++i) { nan |= il[i]; pos_zero |= il2[i]; }
    if (nan) m = NAN;
    else if (m == 0.0f) m = pos_zero ? 0.0f : -0.0f;
  }
  if (m == INFINITY) {
    const float other = log_softmax ? -INFINITY : 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int c = threadIdx.x + i * SM_NT;
      if (c < C4) {
        float4 o;
        o.x = v[i].x == INFINITY ? NAN : other;
        o.y = v[i].y == INFINITY ? NAN : other;
        o.z = v[i].z == INFINITY ? NAN : other;
        o.w = v[i].w == INFINITY ? NAN : other;
        yr[c] = o;
      }
    }
    if (lse != nullptr && threadIdx.x == 0) lse[r] = INFINITY;
    return;
  }
  const bool neg_inf = mn == -INFINITY;
  const float shift = (neg_inf && m == m) ? 0.0f : m;
  // One exponential per element: softmax keeps the rounded addends in registers and scales
  // them by the sum; log-softmax only needs the sum and recomputes x - shift.
  //
  // Every argument x - shift of a row shifted by its finite maximum lies in
  // [fl(min - max), 0] (subtraction rounds monotonically), so when fl(min - max) >= -87 the
  // whole row takes the binary32 path of the exponential without a per-element range test.
  const bool in_range = shift == m && is_finite(m) && mn - m >= -87.0f;  // block-uniform
  float4 e[V];
  float part[V];
  if (in_range) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int c = threadIdx.x + i * SM_NT;
      if (c < C4) {
        e[i].x = exp_f32_in_range(v[i].x - shift);
        e[i].y = exp_f32_in_range(v[i].y - shift);
        e[i].z = exp_f32_in_range(v[i].z - shift);
        e[i].w = exp_f32_in_range(v[i].w - shift);
        part[i] = (e[i].x + e[i].y) + (e[i].z + e[i].w);
      } else {
        part[i] = 0.0f;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int c = threadIdx.x + i * SM_NT;
      if (c < C4) {
        e[i].x = shifted_exp(v[i].x, shift);
        e[i].y = shifted_exp(v[i].y, shift);
        e[i].z = shifted_exp(v[i].z, shift);
        e[i].w = shifted_exp(v[i].w, shift);
        part[i] = (e[i].x + e[i].y) + (e[i].z + e[i].w);
      } else {
        part[i] = 0.0f;
      }
    }
  }
  // Pairwise over the lane's float4 groups (every part is >= 0 or NaN, so zero padding is exact).
#pragma unroll
  for (int h = 1; h < V; h <<= 1)
#pragma unroll
    for (int i = 0; i + h < V; i += 2 * h) part[i] += part[i + h];
  const float sum = (float)block_sum<SM_NT>((double)part[0], dl);
  // Every lane needs the binary64 logarithm of the sum only for log-softmax; softmax needs it
  // only for the LSE output, which lane 0 forms below.
  const float logsum = log_softmax ? (float)log((double)sum) : 0.0f;
  // Softmax scales by the reciprocal of the sum (one division per row; at most one extra
  // rounding per element against the reference's quotient). A sum whose reciprocal would leave
  // the normal range, or a non-finite one, keeps the per-element division.
  const bool recip = sum >= 0x1p-126f && sum <= 0x1p126f;
  const float inv = 1.0f / sum;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + i * SM_NT;
    if (c < C4) {
      float4 o;
      if (log_softmax) {
        o.x = (v[i].x - shift) - logsum;
        o.y = (v[i].y - shift) - logsum;
        o.z = (v[i].z - shift) - logsum;
        o.w = (v[i].w - shift) - logsum;
      } else if (recip) {
        o.x = e[i].x * inv;
        o.y = e[i].y * inv;
        o.z = e[i].z * inv;
        o.w = e[i].w * inv;
      } else {
        o.x = e[i].x / sum;
        o.y = e[i].y / sum;
        o.z = e[i].z / sum;
        o.w = e[i].w / sum;
      }
      st_stream(&yr[c], o);
    }
  }
  if (lse != nullptr) {
    if (neg_inf && is_finite(m)) {
      // LOG_SUM_EXP keeps the maximum as its shift even when the row holds -inf
      // (CpuLogSumExpEmitter.java:4-9); only the softmax values use the unshifted form.
      double s2 = 0.0;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int c = threadIdx.x + i * SM_NT;
        if (c < C4)
          s2 += ((double)shifted_exp(v[i].x, m) + (double)shifted_exp(v[i].y, m)) +
                ((double)shifted_exp(v[i].z, m) + (double)shifted_exp(v[i].w, m));
      }
      const float sum2 = (float)block_sum<SM_NT>(s2, dl);
      if (threadIdx.x == 0) lse[r] = m + (float)log((double)sum2);
    } else if (threadIdx.x == 0) {
      lse[r] = shift + (log_softmax ? logsum : (float)log((double)sum));
    }
  }
}

// Any width: three streaming passes over the row.
__global__ void __launch_bounds__(SM_NT) softmax_fwd_stream(const float* __restrict__ x,
                                                            float* __restrict__ y, float* lse,
                                                            int64_t C, int log_softmax) {
  __shared__ double dl[SM_NT / 64];
  __shared__ float fl[SM_NT / 64];
  __shared__ int il[SM_NT / 64];
  const int64_t r = blockIdx.x;
  const float* xr = x + r * C;
  float* yr = y + r * C;
  float m = -INFINITY;
  int neg_inf = 0;
  for (int64_t c = threadIdx.x; c < C; c += SM_NT) {
    const float t = xr[c];
    m = java_max(m, t);
    neg_inf |= t == -INFINITY;
  }
  m = block_max<SM_NT>(m, fl);
  neg_inf = block_or(neg_inf, il);
  if (m == INFINITY) {
    const float other = log_softmax ? -INFINITY : 0.0f;
    for (int64_t c = threadIdx.x; c < C; c += SM_NT) yr[c] = xr[c] == INFINITY ? NAN : other;
    if (lse != nullptr && threadIdx.x == 0) lse[r] = INFINITY;
    return;
  }
  const float shift = (neg_inf && m == m) ? 0.0f : m;
  double s = 0.0;
  for (int64_t c = threadIdx.x; c < C; c += SM_NT) s += (double)shifted_exp(xr[c], shift);
  const float sum = (float)block_sum<SM_NT>(s, dl);
  const float logsum = (float)log((double)sum);
  for (int64_t c = threadIdx.x; c < C; c += SM_NT)
    yr[c] = log_softmax ? (xr[c] - shift) - logsum : shifted_exp(xr[c], shift) / sum;
  if (lse != nullptr) {
    float l = C == 0 ? -INFINITY : shift + logsum;
    if (neg_inf && is_finite(m)) {  // LOG_SUM_EXP shifts by the maximum (see above)
      double s2 = 0.0;
      for (int64_t c = threadIdx.x; c < C; c += SM_NT) s2 += (double)shifted_exp(xr[c], m);
      l = m + (float)log((double)(float)block_sum<SM_NT>(s2, dl));
    }
    if (threadIdx.x == 0) lse[r] = l;
  }
}

// dX = y (.) (g - s) [+ k_r * y], s = sum(g (.) y)  (ReductionGradientRules.java:84-90).
template <int V>
__global__ void __launch_bounds__(SM_NT) softmax_bwd_regs(const float* __restrict__ y,
                                                          const float* __restrict__ g,
                                                          float* __restrict__ dx, int64_t C,
                                                          const float* rowscale, float rsc) {
  __shared__ double dl[SM_NT / 64];
  const int64_t r = blockIdx.x;
  const float4* yr = reinterpret_cast<const float4*>(y + r * C);
  const float4* gr = reinterpret_cast<const float4*>(g + r * C);
  float4* dr = reinterpret_cast<float4*>(dx + r * C);
  const int C4 = (int)(C / 4);
  float4 yv[V], gv[V];
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + i * SM_NT;
    if (c < C4) {
      yv[i] = ld_stream(&yr[c]);
      gv[i] = ld_stream(&gr[c]);
      s += (double)(gv[i].x * yv[i].x);
      s += (double)(gv[i].y * yv[i].y);
      s += (double)(gv[i].z * yv[i].z);
      s += (double)(gv[i].w * yv[i].w);
    }
  }
  const float sf = (float)block_sum<SM_NT>(s, dl);
  const bool scaled = rowscale != nullptr || rsc != 0.0f;
  const float k = rowscale != nullptr ? rowscale[r] : rsc;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + i * SM_NT;
    if (c < C4) {
      float4 o;
      o.x = yv[i].x * (gv[i].x - sf);
      o.y = yv[i].y * (gv[i].y - sf);
      o.z = yv[i].z * (gv[i].z - sf);
      o.w = yv[i].w * (gv[i].w - sf);
      if (scaled) {
        o.x = o.x + k * yv[i].x;
        o.y = o.y + k * yv[i].y;
        o.z = o.z + k * yv[i].z;
        o.w = o.w + k * yv[i].w;
      }
      st_stream(&dr[c], o);
    }
  }
}

__global__ void __launch_bounds__(SM_NT) softmax_bwd_stream(const float* __restrict__ y,
                                                            const float* __restrict__ g,
                                                            float* __restrict__ dx, int64_t C,
                                                            const float* rowscale, float rsc) {
  __shared__ double dl[SM_NT / 64];
  const int64_t r = blockIdx.x;
  const float* yr = y + r * C;
  const float* gr = g + r * C;
  float* dr = dx + r * C;
  double s = 0.0;
  for (int64_t c = threadIdx.x; c < C; c += SM_NT) s += (double)(gr[c] * yr[c]);
  const float sf = (float)block_sum<SM_NT>(s, dl);
  const bool scaled = rowscale != nullptr || rsc != 0.0f;
  const float k = rowscale != nullptr ? rowscale[r] : rsc;
  for (int64_t c = threadIdx.x; c < C; c += SM_NT) {
    float o = yr[c] * (gr[c] - sf);
    if (scaled) o = o + k * yr[c];
    dr[c] = o;
  }
}

// LOG_SUM_EXP gradient g_r * exp(x - lse_r) (ReductionGradientRules.java:213-224).
__global__ void lse_bwd_kernel(const float* __restrict__ x, const float* __restrict__ lse,
                               const float* g, float gconst, float* __restrict__ dx, int64_t R,
                               int64_t C) {
  const int64_t n = R * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / C;
    const float gr = g != nullptr ? g[r] : gconst;
    dx[i] = gr * (float)exp((double)(x[i] - lse[r]));
  }
}

// ---- MSE (CpuLossReferenceKernel.java:67-87, LossGradientRules.java:77-97) ----
constexpr int MSE_BLOCKS = 1024;
// MEAN finalization divides the binary32 sum by the exact count before one final rounding.
__device__ __forceinline__ float mse_loss(double s, int64_t n, int reduction_sum) {
  const float sf = (float)s;
  return reduction_sum ? sf : (float)((double)sf / (double)n);
}
// Pass 1: block b's binary64 partial sum of squared differences (and the gradient). A launch of
// one block finishes the loss itself: its partial is the whole sum, which pass 2 would only
// return unchanged.
__global__ void __launch_bounds__(256) mse_pass1(const float* __restrict__ p,
                                                 const float* __restrict__ t,
                                                 float* __restrict__ grad, int64_t n, float gn,
                                                 double* part, float* loss, int reduction_sum) {
  __shared__ double dl[4];
  double s = 0.0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(t) |
                     reinterpret_cast<uintptr_t>(grad)) & 15u) == 0;
  int64_t head = 0;
  if (vec) {
    // four elements per thread and iteration, streaming 16-byte accesses
    const int64_t n4 = n / 4;
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n4; q += stride) {
      const float4 pv = ld_stream(reinterpret_cast<const float4*>(p) + q);
      const float4 tv = ld_stream(reinterpret_cast<const float4*>(t) + q);
      const float d0 = pv.x - tv.x, d1 = pv.y - tv.y, d2 = pv.z - tv.z, d3 = pv.w - tv.w;
      const float q0 = d0 * d0, q1 = d1 * d1, q2 = d2 * d2, q3 = d3 * d3;
      s += ((double)q0 + (double)q1) + ((double)q2 + (double)q3);
      if (grad != nullptr) {
        const float t0 = d0 * 2.0f, t1 = d1 * 2.0f, t2 = d2 * 2.0f, t3 = d3 * 2.0f;
        st_stream(reinterpret_cast<float4*>(grad) + q, make_float4(t0 * gn, t1 * gn, t2 * gn, t3 * gn));
      }
    }
    head = n4 * 4;
  }
  for (int64_t i = head + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const float d = p[i] - t[i];
    const float sq = d * d;
    s += (double)sq;
    if (grad != nullptr) {
      const float twice = d * 2.0f;
      grad[i] = twice * gn;
    }
  }
  s = block_sum<256>(s, dl);
  if (threadIdx.x == 0) {
    if (gridDim.x == 1) loss[0] = mse_loss(s, n, reduction_sum);
    else part[blockIdx.x] = s;
  }
}
__global__ void __launch_bounds__(256) mse_pass2(const double* part, int P, int64_t n,
                                                 int reduction_sum, float* loss) {
  __shared__ double dl[4];
  double s = 0.0;
  for (int i = threadIdx.x; i < P; i += 256) s += part[i];
  s = block_sum<256>(s, dl);
  if (threadIdx.x == 0) loss[0] = mse_loss(s, n, reduction_sum);
}

// ---- Index categorical cross-entropy (CpuLossReferenceKernel.java:196-218,261-288;
//      LossGradientRules.java:172-240). One wave per sample row. ----
template <typename T>
__global__ void __launch_bounds__(256) ce_pass1(const float* __restrict__ logits,
                                                const T* __restrict__ target, int64_t R,
                                                int64_t C, int has_ignore, int64_t ignore,
                                                double* part, uint32_t* status) {
  __shared__ double dl[4];
  __shared__ double dc[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * 4 + w;
  double loss = 0.0, count = 0.0;
  if (r < R) {
    const int64_t t = (int64_t)target[r];
    const bool ignored = has_ignore && t == ignore;
    if (!ignored) {
      if (t < 0 || t >= C) {
        if (lane == 0) atomicOr(status, (uint32_t)DEV_INDEX_OUT_OF_BOUNDS);
      } else {
        const float* row = logits + r * C;
        // maximum by '>' (a NaN logit never becomes the maximum), as the loss oracle does
        float m = -INFINITY;
        for (int64_t c = lane; c < C; c += 64) {
          const float v = row[c];
          if (v > m) m = v;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float u = __shfl_xor(m, o, 64);
          if (u > m) m = u;
        }
        double s = 0.0;
        for (int64_t c = lane; c < C; c += 64) s += (double)(float)exp((double)(row[c] - m));
        s = wave_sum(s);
        const float lse = m + (float)log((double)(float)s);
        loss = (double)(lse - row[t]);
        count = 1.0;
      }
    }
  }
  if (lane != 0) { loss = 0.0; count = 0.0; }
  if (lane == 0) { dl[w] = loss; dc[w] = count; }
  __syncthreads();
  if (threadIdx.x == 0) {
    part[2 * blockIdx.x] = ((dl[0] + dl[1]) + dl[2]) + dl[3];
    part[2 * blockIdx.x + 1] = ((dc[0] + dc[1]) + dc[2]) + dc[3];
  }
}
__device__ __forceinline__ void ce_finish(double* part, int P, float* loss, double* dl) {
  double s = 0.0, c = 0.0;
  for (int i = threadIdx.x; i < P; i += 256) {
    s += part[2 * i];
    c += part[2 * i + 1];
  }
  s = block_sum<256>(s, dl);
  __syncthreads();
  c = block_sum<256>(c, dl);
  if (threadIdx.x == 0) {
    loss[0] = (float)s / (float)c;
    part[2 * P] = c;  // non-ignored sample count for the gradient pass
  }
}
__global__ void __launch_bounds__(256) ce_pass2(double* part, int P, float* loss) {
  __shared__ double dl[4];
  ce_finish(part, P, loss, dl);
}
// Gradient rows. FUSED: the launch is the one after ce_pass1 (no ce_pass2): block 0 first does
// ce_pass2's work (same code, same order), and every block sums the P exact per-block sample
// counts itself (integers in binary64, exact in any order) instead of reading the total.
template <typename T, bool FUSED>
__global__ void __launch_bounds__(256) ce_grad(const float* __restrict__ logits,
                                               const T* __restrict__ target, int64_t R, int64_t C,
                                               int has_ignore, int64_t ignore, float g,
                                               double* part, int P, float* loss,
                                               float* __restrict__ grad) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  double count;
  if (FUSED) {
    __shared__ double dl[4];
    if (blockIdx.x == 0) {
      ce_finish(part, P, loss, dl);
      __syncthreads();
    }
    double c = 0.0;
    for (int i = threadIdx.x; i < P; i += 256) c += part[2 * i + 1];
    count = block_sum<256>(c, dl);
  } else {
    count = part[2 * P];
  }
  const int64_t r = (int64_t)blockIdx.x * 4 + w;
  if (r >= R) return;
  const int64_t t = (int64_t)target[r];
  const float* row = logits + r * C;
  float* gr = grad + r * C;
  if (has_ignore && t == ignore) {
    for (int64_t c = lane; c < C; c += 64) gr[c] = 0.0f;
    return;
  }
  const float scale = g / (float)count;
  const int64_t safe = t < 0 ? 0 : (t >= C ? C - 1 : t);
  float m = -INFINITY;
  for (int64_t c = lane; c < C; c += 64) m = java_max(m, row[c]);
  m = wave_max(m);
  double s = 0.0;
  for (int64_t c = lane; c < C; c += 64) s += (double)(float)exp((double)(row[c] - m));
  const float sum = (float)wave_sum(s);
  for (int64_t c = lane; c < C; c += 64) {
    const float prob = (float)exp((double)(row[c] - m)) / sum;
    const float hot = c == safe ? 1.0f : 0.0f;
    gr[c] = (prob - hot) * scale;
  }
}

}  // namespace

hipError_t launch_softmax_fwd(const float* x, float* y, float* lse, int64_t R, int64_t C,
                              int log_softmax, hipStream_t s) {
  if (R <= 0) return hipSuccess;
  const bool vec = C % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
  dim3 g((unsigned)R), b(SM_NT);
  if (vec && C > 0 && C <= 1024)
    hipLaunchKernelGGL(softmax_fwd_regs<1>, g, b, 0, s, x, y, lse, C, log_softmax);
  else if (vec && C > 0 && C <= 2048)
    hipLaunchKernelGGL(softmax_fwd_regs<2>, g, b, 0, s, x, y, lse, C, log_softmax);
  else if (vec && C > 0 && C <= 4096)
    hipLaunchKernelGGL(softmax_fwd_regs<4>, g, b, 0, s, x, y, lse, C, log_softmax);
  else
    hipLaunchKernelGGL(softmax_fwd_stream, g, b, 0, s, x, y, lse, C, log_softmax);
  return hipGetLastError();
}

hipError_t launch_softmax_bwd(const float* y, const float* g, float* dx, int64_t R, int64_t C,
                              const float* rowscale, float rowscale_const, hipStream_t s) {
  if (R <= 0) return hipSuccess;
  const bool vec = C % 4 == 0 &&
      ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(g) |
        reinterpret_cast<uintptr_t>(dx)) & 15u) == 0;
  dim3 gr((unsigned)R), b(SM_NT);
  if (vec && C > 0 && C <= 1024)
    hipLaunchKernelGGL(softmax_bwd_regs<1>, gr, b, 0, s, y, g, dx, C, rowscale, rowscale_const);
  else if (vec && C > 0 && C <= 2048)
    hipLaunchKernelGGL(softmax_bwd_regs<2>, gr, b, 0, s, y, g, dx, C, rowscale, rowscale_const);
  else if (vec && C > 0 && C <= 4096)
    hipLaunchKernelGGL(softmax_bwd_regs<4>, gr, b, 0, s, y, g, dx, C, rowscale, rowscale_const);
  else
    hipLaunchKernelGGL(softmax_bwd_stream, gr, b, 0, s, y, g, dx, C, rowscale, rowscale_const);
  return hipGetLastError();
}

hipError_t launch_lse_bwd(const float* x, const float* lse, const float* g, float gconst,
                          float* dx, int64_t R, int64_t C, hipStream_t s) {
  const int64_t n = R * C;
  if (n <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<int64_t>(65536, (n + 255) / 256);
  hipLaunchKernelGGL(lse_bwd_kernel, dim3(blocks), dim3(256), 0, s, x, lse, g, gconst, dx, R, C);
  return hipGetLastError();
}

int64_t mse_partial_doubles(int64_t) { return MSE_BLOCKS; }
hipError_t launch_mse(const float* p, const float* t, float* loss, float* grad, int64_t n,
                      float g, int reduction_sum, double* partial, hipStream_t s) {
  const unsigned blocks = (unsigned)std::min<int64_t>(MSE_BLOCKS, std::max<int64_t>(1, (n + 1023) / 1024));
  // restore(g): MEAN divides g by the count (an exact binary32 sum of ones); SUM expands g.
  const float gn = reduction_sum ? g : g / (float)n;
  hipLaunchKernelGGL(mse_pass1, dim3(blocks), dim3(256), 0, s, p, t, grad, n, gn, partial, loss,
                     reduction_sum);
  if (blocks > 1)
    hipLaunchKernelGGL(mse_pass2, dim3(1), dim3(256), 0, s, (const double*)partial, (int)blocks,
                       n, reduction_sum, loss);
  return hipGetLastError();
}

constexpr unsigned CE_FUSE_BLOCKS = 1024;
int64_t index_ce_partial_doubles(int64_t R) { return 2 * ((R + 3) / 4) + 2; }
hipError_t launch_index_ce(const float* logits, const void* target, int target_is_64,
                           float* loss, float* grad, int64_t R, int64_t C, int has_ignore,
                           int64_t ignore_index, float g, double* partial, uint32_t* status,
                           hipStream_t s) {
  if (R <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)((R + 3) / 4);
  if (target_is_64)
    hipLaunchKernelGGL(ce_pass1<int64_t>, dim3(blocks), dim3(256), 0, s, logits,
                       (const int64_t*)target, R, C, has_ignore, ignore_index, partial, status);
  else
    hipLaunchKernelGGL(ce_pass1<int32_t>, dim3(blocks), dim3(256), 0, s, logits,
                       (const int32_t*)target, R, C, has_ignore, ignore_index, partial, status);
  const int P = (int)blocks;
  // Up to CE_FUSE_BLOCKS blocks, the gradient launch also finishes the loss (each block re-sums
  // the P counts: 2P doubles read per block); beyond that a separate one-block pass does.
  const bool fuse = grad != nullptr && blocks <= CE_FUSE_BLOCKS;
  if (!fuse) hipLaunchKernelGGL(ce_pass2, dim3(1), dim3(256), 0, s, partial, P, loss);
  if (grad != nullptr) {
    if (target_is_64) {
      if (fuse)
        hipLaunchKernelGGL((ce_grad<int64_t, true>), dim3(blocks), dim3(256), 0, s, logits,
                           (const int64_t*)target, R, C, has_ignore, ignore_index, g, partial, P,
                           loss, grad);
      else
        hipLaunchKernelGGL((ce_grad<int64_t, false>), dim3(blocks), dim3(256), 0, s, logits,
                           (const int64_t*)target, R, C, has_ignore, ignore_index, g, partial, P,
                           loss, grad);
    } else {
      if (fuse)
        hipLaunchKernelGGL((ce_grad<int32_t, true>), dim3(blocks), dim3(256), 0, s, logits,
                           (const int32_t*)target, R, C, has_ignore, ignore_index, g, partial, P,
                           loss, grad);
      else
        hipLaunchKernelGGL((ce_grad<int32_t, false>), dim3(blocks), dim3(256), 0, s, logits,
                           (const int32_t*)target, R, C, has_ignore, ignore_index, g, partial, P,
                           loss, grad);
    }
  }
  return hipGetLastError();
}

}  // namespace shk
