// Fused classifier head for training: logits, index cross-entropy and both cotangents in one pass
// over the head's input rows.
//
// For a last layer with J <= 16 classes (logits = H . W^T + b, H [R, K], W [J, K]) followed by
// MEAN index cross-entropy without an ignore index, one wave owns one row r and computes
//   logits[r, :]   as gemm_row_dot does: lanes split k in 16-byte steps (fmaf over x, y, z, w),
//                  the transpose-reduce butterfly over the wave, then + b (the GEMM epilogue);
//   row_loss[r]    lse - logits[r, t] with the maximum by '>' and the binary64 wave sum of the
//                  rounded exponentials, as ce_pass1 does (CpuLossReferenceKernel.java:196-218);
//   dZ[r, :]       (softmax - onehot(t)) * (g / R), the maximum by Math.max, as ce_grad does
//                  (LossGradientRules.java:172-240);
//   dX[r, :]       act_grad(act, dZ[r, :] . W, H[r, :]), each output an fmaf chain over j from +0,
//                  as gemm_small_k does with the activation-gradient epilogue.
// Every value is the one the unfused sequence (row-dot GEMM, CE pass 1 and gradient, small-K
// GEMM) produces, bit for bit: the fusion removes three launches and the logits round trip from
// the critical path of the backward sweep, nothing else. A second launch (phase 1) finishes the
// MEAN from the per-row losses with ce_pass1 / ce_finish's grouping: binary64 partials of four
// consecutive rows, summed over groups in a strided order and a block tree, divided by R.
#include "common.h"
#include "gemm_tile.h"
#include "kernels.h"

#include <type_traits>

namespace shk {
namespace {

__device__ __forceinline__ float comp(const float4& v, int c) {
  return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}

constexpr int64_t CE_HEAD_LDS_BYTES = 64 * 1024;
constexpr int CE_HEAD_LDS_F4 = (int)(CE_HEAD_LDS_BYTES / 16);

// W is read by every row: with LDSW the block first copies it (J x K, 16-byte aligned, at most
// CE_HEAD_LDS_BYTES) into LDS, so the four waves read it from there instead of from L2 twice
// each. The bucket's padding rows (j >= J) read row J - 1 again and their sums are dropped, as
// in the row-dot kernel: loads and selects without branches keep the LDS reads in flight together.
template <typename T, int JB, bool LDSW>
__global__ void __launch_bounds__(256) ce_head_rows(CeHeadParams p) {
  extern __shared__ float4 wlds[];
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int J = p.J;
  const int64_t K = p.K;
  const float* W = p.W;
  const bool row_ok = r < p.R;
  const float* h = p.H + (row_ok ? r : 0) * K;
  // The row's first HC float4 per lane (K <= 1024) stay in registers from the logits pass to the mask of the
  // input cotangent; their loads are issued before the block waits for W.
  constexpr int HC = 4;
  float4 hv[HC];
  if (p.vec) {
#pragma unroll
    for (int i = 0; i < HC; ++i) {
      const int64_t k = 4 * lane + 256 * i;
      if (k < K) hv[i] = *reinterpret_cast<const float4*>(h + k);
    }
  }
  // the target and the bias are needed only after the logits: their loads go out now
  const int64_t t = row_ok ? (int64_t)static_cast<const T*>(p.target)[r] : 0;
  const float bj = p.bias != nullptr ? p.bias[lane < J ? lane : J - 1] : 0.0f;
  if (LDSW) {
    // W is J x K floats, a multiple of 16 bytes: 1 KB chunks go global -> LDS directly
    // (global_load_lds_dwordx4: lane l's 16 bytes land at M0 + 16 l), all of a wave's chunks in
    // flight at once; the last partial chunk is issued by the lanes it covers. The copies are not
    // tracked by the compiler: the wave waits for them (vmcnt) before the barrier.
    const int64_t n4 = (int64_t)J * K / 4;
    const int64_t chunks = (n4 + 63) / 64;
    const int w = threadIdx.x >> 6;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float4*)wlds;
    for (int64_t c = w; c < chunks; c += 4) {
      if (c * 64 + lane < n4) {
        const uint32_t voff = (uint32_t)((c * 64 + lane) * 16);
        asm volatile("global_load_lds_dwordx4 %0, %1"
                     :
                     : "v"(voff), "s"(p.W), "{m0}"(lds0 + (uint32_t)(c * 1024))
                     : "memory");
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    W = reinterpret_cast<const float*>(wlds);
  }
  if (!row_ok) return;
  // ---- logits: per-lane partial dots, then the transpose-reduce ----
  float acc[JB];
#pragma unroll
  for (int j = 0; j < JB; ++j) acc[j] = 0.0f;
  if (p.vec) {
    auto dot = [&](int64_t k, const float4& xv) {
      float4 yv[JB];
#pragma unroll
      for (int j = 0; j < JB; ++j)
        yv[j] = *reinterpret_cast<const float4*>(W + (j < J ? j : J - 1) * K + k);
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        acc[j] = fmaf(xv.x, yv[j].x, acc[j]);
        acc[j] = fmaf(xv.y, yv[j].y, acc[j]);
        acc[j] = fmaf(xv.z, yv[j].z, acc[j]);
        acc[j] = fmaf(xv.w, yv[j].w, acc[j]);
      }
    };
#pragma unroll
    for (int i = 0; i < HC; ++i)
      if (4 * lane + 256 * i < K) dot(4 * lane + 256 * i, hv[i]);
    for (int64_t k = 4 * lane + 256 * HC; k < K; k += 256)
      dot(k, *reinterpret_cast<const float4*>(h + k));
  } else {
#pragma unroll 2
    for (int64_t k = lane; k < K; k += 64) {
      const float xv = h[k];
      float yv[JB];
#pragma unroll
      for (int j = 0; j < JB; ++j) yv[j] = W[(j < J ? j : J - 1) * K + k];
#pragma unroll
      for (int j = 0; j < JB; ++j) acc[j] = fmaf(xv, yv[j], acc[j]);
    }
  }
  constexpr int LG = JB == 1 ? 0 : JB == 2 ? 1 : JB == 4 ? 2 : JB == 8 ? 3 : 4;
  static_for<LG>([&](auto round) {
    constexpr int RD = decltype(round)::value;
    constexpr int H = JB >> (RD + 1);
    const int off = 32 >> RD;
    const bool upper = (lane & off) != 0;
#pragma unroll
    for (int j = 0; j < H; ++j) {
      const float send = upper ? acc[j] : acc[j + H];
      const float keep = upper ? acc[j + H] : acc[j];
      acc[j] = keep + __shfl_xor(send, off, 64);
    }
  });
#pragma unroll
  for (int off = 32 >> LG; off >= 1; off >>= 1) acc[0] += __shfl_xor(acc[0], off, 64);
  // lane j (< J) takes logit j from the lane group that holds it, then the bias
  const bool cls = lane < J;
  const int jl = cls ? lane : J - 1;
  float z = __shfl(acc[0], jl << (6 - LG), 64);
  if (p.bias != nullptr) z = z + bj;
  if (p.logits != nullptr && cls) p.logits[r * J + lane] = z;

  // ---- cross-entropy: one class per lane ----
  const bool in_range = t >= 0 && t < J;
  if (!in_range && lane == 0) atomicOr(p.status, (uint32_t)DEV_INDEX_OUT_OF_BOUNDS);
  const float zt = __shfl(z, in_range ? (int)t : 0, 64);
  // The loss shifts by the maximum by '>' (a NaN logit never becomes the maximum), the gradient
  // by Math.max. Without a NaN the two agree up to the sign of a zero maximum, which changes no
  // shifted value's exponential, so one set of rounded exponentials serves both sums.
  // Classes occupy lanes 0 .. 15; the 64-lane butterflies of the unfused kernels only fold
  // padding (-inf for maxima, +0 for the sums of non-negative terms) into those lanes in their
  // first two rounds, so butterflies over 16 lanes give the same values.
  float m = cls ? z : -INFINITY;
  if (!(m > -INFINITY)) m = -INFINITY;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) {
    const float u = __shfl_xor(m, o, 64);
    if (u > m) m = u;
  }
  float m2 = cls ? z : -INFINITY;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) m2 = java_max(m2, __shfl_xor(m2, o, 64));
  auto sum16 = [](double v) {
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
  };
  const float e2 = cls ? (float)exp((double)(z - m2)) : 0.0f;
  const double s2 = sum16(cls ? (double)e2 : 0.0);
  const float sum2 = (float)s2;
  double s = s2;
  if (!(m == m2)) s = sum16(cls ? (double)(float)exp((double)(z - m)) : 0.0);  // a NaN logit
  const float lse = m + (float)log((double)(float)s);
  if (lane == 0) p.row_loss[r] = in_range ? lse - zt : 0.0f;
  const int64_t safe = t < 0 ? 0 : (t >= J ? J - 1 : t);
  const float scale = p.g / (float)(double)p.R;
  float dz = 0.0f;
  if (cls) {
    const float prob = e2 / sum2;
    const float hot = lane == safe ? 1.0f : 0.0f;
    dz = (prob - hot) * scale;
    p.dz[r * J + lane] = dz;
  }
  if (p.dx == nullptr) return;

  // ---- dX = act_grad(dZ . W, H): every lane holds all J cotangents ----
  float d[JB];
#pragma unroll
  for (int j = 0; j < JB; ++j)
    d[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dz), j < J ? j : J - 1));
  float* dxr = p.dx + r * K;
  // one loop per activation (the switch is outside it: branches inside would make every LDS
  // read wait for the one before)
  auto dx_rows = [&](auto actc) {
    constexpr int A = decltype(actc)::value;
    if (p.vec) {
      auto out = [&](int64_t k, const float4& y) {
        float4 w[JB];
#pragma unroll
        for (int j = 0; j < JB; ++j)
          w[j] = *reinterpret_cast<const float4*>(W + (j < J ? j : J - 1) * K + k);
        float o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float sum = fmaf(d[0], comp(w[0], c), 0.0f);
#pragma unroll
          for (int j = 1; j < JB; ++j) {
            const float tt = fmaf(d[j], comp(w[j], c), sum);
            sum = j < J ? tt : sum;
          }
          o[c] = sum;
        }
        *reinterpret_cast<float4*>(dxr + k) =
            make_float4(act_grad(A, o[0], y.x), act_grad(A, o[1], y.y), act_grad(A, o[2], y.z),
                        act_grad(A, o[3], y.w));
      };
#pragma unroll
      for (int i = 0; i < HC; ++i)
        if (4 * lane + 256 * i < K) out(4 * lane + 256 * i, hv[i]);
      for (int64_t k = 4 * lane + 256 * HC; k < K; k += 256)
        out(k, *reinterpret_cast<const float4*>(h + k));
    } else {
      for (int64_t k = lane; k < K; k += 64) {
        float sum = fmaf(d[0], W[k], 0.0f);
#pragma unroll
        for (int j = 1; j < JB; ++j) {
          const float tt = fmaf(d[j], W[(j < J ? j : J - 1) * K + k], sum);
          sum = j < J ? tt : sum;
        }
        dxr[k] = act_grad(A, sum, h[k]);
      }
    }
  };
  switch (p.act) {
    case ACT_RELU: dx_rows(std::integral_constant<int, ACT_RELU>{}); break;
    case ACT_TANH: dx_rows(std::integral_constant<int, ACT_TANH>{}); break;
    case ACT_SIGMOID: dx_rows(std::integral_constant<int, ACT_SIGMOID>{}); break;
    default: dx_rows(std::integral_constant<int, ACT_NONE>{}); break;
  }
}

__global__ void __launch_bounds__(256) ce_head_finish(const float* __restrict__ row_loss, int64_t R,
                                                      float* loss) {
  __shared__ double dl[4];
  ce_mean_block(row_loss, R, loss, dl);
}

template <typename T, bool LDSW>
hipError_t launch_rows_w(const CeHeadParams& p, size_t lds, hipStream_t s) {
  const dim3 g((unsigned)((p.R + 3) / 4)), b(256);
  switch (p.J <= 1 ? 1 : p.J <= 2 ? 2 : p.J <= 4 ? 4 : p.J <= 8 ? 8 : 16) {
    case 1: hipLaunchKernelGGL((ce_head_rows<T, 1, LDSW>), g, b, lds, s, p); break;
    case 2: hipLaunchKernelGGL((ce_head_rows<T, 2, LDSW>), g, b, lds, s, p); break;
    case 4: hipLaunchKernelGGL((ce_head_rows<T, 4, LDSW>), g, b, lds, s, p); break;
    case 8: hipLaunchKernelGGL((ce_head_rows<T, 8, LDSW>), g, b, lds, s, p); break;
    default: hipLaunchKernelGGL((ce_head_rows<T, 16, LDSW>), g, b, lds, s, p); break;
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_rows(const CeHeadParams& p, hipStream_t s) {
  const int64_t wbytes = (int64_t)p.J * p.K * 4;
  if (p.vec && wbytes <= CE_HEAD_LDS_BYTES) return launch_rows_w<T, true>(p, (size_t)wbytes, s);
  return launch_rows_w<T, false>(p, 0, s);
}

}  // namespace

hipError_t launch_ce_head(const CeHeadParams& in, hipStream_t s) {
  if (in.R <= 0) return hipSuccess;
  CeHeadParams p = in;
  p.vec = p.K % 4 == 0 &&
          ((reinterpret_cast<uintptr_t>(p.H) | reinterpret_cast<uintptr_t>(p.W) |
            reinterpret_cast<uintptr_t>(p.dx)) & 15u) == 0;
  return p.target_is_64 ? launch_rows<int64_t>(p, s) : launch_rows<int32_t>(p, s);
}

hipError_t launch_ce_head_finish(const float* row_loss, int64_t R, float* loss, hipStream_t s) {
  if (R <= 0) return hipSuccess;
  hipLaunchKernelGGL(ce_head_finish, dim3(1), dim3(256), 0, s, row_loss, R, loss);
  return hipGetLastError();
}

}  // namespace shk
