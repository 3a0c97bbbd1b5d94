// fp32 MFMA GEMM for gfx950 (CDNA4): C = op(A) . op(B) with fused bias/activation epilogue.
//
// Replaces the reference's MATMUL routes for the Linear path:
//   forward  Z = X . W^T          (TensorLinearExpressions.java:97-146)        -> transB = 1
//   backward dX = dZ . W          (LinearAlgebraGradientRules.java:97-104)     -> NN
//   backward dW = PERMUTE(X^T.dZ) (LayoutGradientRules.java:114), written directly as
//            dW[out,in] = dZ^T . X                                             -> transA = 1
// The reference contract allows a backend to reassociate an operation's reduction and use
// FP32 FMA within one operation (docs/architecture/contracts/foundational-modules.md:423-425),
// which is what the matrix cores do; results differ from the sequential no-FMA CPU oracle only
// by reduction order (and are bit-identical when all partial sums are exact).
//
// Design (one workgroup per BM x BN output tile):
//   * v_mfma_f32_32x32x2_f32: each wave owns a WM x WN sub-tile as (WM/32) x (WN/32)
//     32x32 accumulator blocks (16 fp32 accumulators per lane per block).
//   * Both operand tiles are staged through LDS in a [k][m] / [k][n] layout (m/n contiguous,
//     padded pitch) so that every MFMA operand fetch is one conflict-light ds_read_b32 with
//     consecutive lanes on consecutive addresses; K-contiguous global operands are transposed
//     on the way in, M/N-contiguous ones are stored with ds_write_b128.
//   * LDS is double buffered: the global loads of tile k+1 are issued into registers before the
//     MFMAs of tile k, and written to the other LDS buffer afterwards (one barrier per tile).
//   * Workgroup ids are remapped so that each of the 8 XCDs receives a contiguous, M-grouped
//     block of output tiles: tiles that share A row-panels and B column-panels share an L2.
//
// The tile kernel lives in gemm_tile.h and is instantiated per operand layout in gemm_nn.hip,
// gemm_nt.hip, gemm_tn.hip and gemm_tt.hip; this file holds the dispatch, the deterministic
// split-K reduction and the K == 1 outer product.
#include "gemm_skinny.h"
#include "gemm_tile.h"
#include "gemm_v2.h"
#include <algorithm>

namespace shk {

thread_local int64_t g_colsum_rows = 0;

namespace {
// K == 1: every output is exactly one product a*b (CpuMatmulReferenceKernel.java:34-119: a
// singleton contraction is one typed product, no identity ADD), which keeps the sign of a zero
// product; the MFMA path would add it to a +0 accumulator. Same epilogue as the MFMA kernel.
__global__ void __launch_bounds__(256) gemm_k1_outer(GemmParams p) {
  const int64_t total = p.M * p.N;
  const bool upd = p.upd.pn != nullptr;
  UpdateCtx uc{};
  bool ok = true;
  if (upd) {
    uc = update_ctx(p.upd);
    ok = uc.k.ok;
  }
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t row = e / p.N, col = e - row * p.N;
    const float a = p.A[row * (p.transA ? 1 : p.lda)];
    const float b = p.B[col * (p.transB ? p.ldb : 1)];
    float v = a * b;
    if (upd) {
      ok &= update_scalar(p.upd, uc, e, v);
      continue;
    }
    if (p.mode == 0) {
      if (p.bias != nullptr) v = v + p.bias[col];
      v = apply_act(p.act, v);
    } else {
      v = act_grad(p.act, v, p.aux[row * p.ldaux + col]);
    }
    float* dst = p.C + row * p.ldc + col;
    if (p.accumulate) v = *dst + v;
    *dst = v;
  }
  if (upd) update_flag(p.upd, uc, ok);
}

// dz = act_grad(act, dy, y) over an [M, N] view (dy and dz with leading dimension ld, y with ldy):
// the second output of a forward GEMM with its cotangent (mode 2) on routes whose epilogue does
// not form it.
__global__ void __launch_bounds__(256) gemm_cotangent_pass(const float* __restrict__ y, int64_t ldy,
                                                           const float* __restrict__ dy,
                                                           float* __restrict__ dz, int64_t ld,
                                                           int64_t M, int64_t N, int act) {
  const int64_t total = M * N;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t row = e / N, col = e - row * N;
    dz[row * ld + col] = act_grad(act, dy[row * ld + col], y[row * ldy + col]);
  }
}

// Split-K reduction: sums the slices of each output in slice order (a fixed binary32 order, so
// results are deterministic) and applies the GEMM epilogue.
__global__ void __launch_bounds__(256) gemm_splitk_reduce(GemmParams p, int splits) {
  const int64_t total = p.M * p.N;
  const int64_t plane = total;
  const bool upd = p.upd.pn != nullptr;
  UpdateCtx uc{};
  bool ok = true;
  if (upd) {
    uc = update_ctx(p.upd);
    ok = uc.k.ok;
  }
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t row = e / p.N, col = e - row * p.N;
    float v = p.partial[e];
    int sidx = 1;
    for (; sidx + 8 <= splits; sidx += 8) {  // eight loads in flight, added in slice order
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = p.partial[(sidx + u) * plane + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) v = v + t[u];
    }
    for (; sidx < splits; ++sidx) v = v + p.partial[sidx * plane + e];
    if (upd) {
      ok &= update_scalar(p.upd, uc, e, v);
      continue;
    }
    if (p.mode == 0) {
      if (p.bias != nullptr) v = v + p.bias[col];
      v = apply_act(p.act, v);
    } else {
      v = act_grad(p.act, v, p.aux[row * p.ldaux + col]);
    }
    float* dst = p.C + row * p.ldc + col;
    if (p.accumulate) v = *dst + v;
    *dst = v;
  }
  if (upd) update_flag(p.upd, uc, ok);
}

// The same reduction four consecutive outputs at a time (N, ldc, ldaux multiples of 4 and every
// pointer 16-byte aligned): float4 loads of the slices and float4 epilogue traffic.
__global__ void __launch_bounds__(256) gemm_splitk_reduce4(GemmParams p, int splits) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int64_t groups = p.M * p.N / 4;
  const int64_t plane = p.M * p.N;
  const bool upd = p.upd.pn != nullptr;
  UpdateCtx uc{};
  bool ok = true;
  if (upd) {
    uc = update_ctx(p.upd);
    ok = uc.k.ok;
  }
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < groups; q += (int64_t)gridDim.x * 256) {
    const int64_t e = 4 * q, row = e / p.N, col = e - row * p.N;
    f4 v = *reinterpret_cast<const f4*>(p.partial + e);
    int sidx = 1;
    for (; sidx + 4 <= splits; sidx += 4) {  // four loads in flight, added in slice order
      f4 t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) t[u] = *reinterpret_cast<const f4*>(p.partial + (sidx + u) * plane + e);
#pragma unroll
      for (int u = 0; u < 4; ++u) v = f4{v[0] + t[u][0], v[1] + t[u][1], v[2] + t[u][2], v[3] + t[u][3]};
    }
    for (; sidx < splits; ++sidx) {
      const f4 w = *reinterpret_cast<const f4*>(p.partial + sidx * plane + e);
      v = f4{v[0] + w[0], v[1] + w[1], v[2] + w[2], v[3] + w[3]};
    }
    if (upd) {
      const GemmUpdate& u = p.upd;
      const f4 pv = *reinterpret_cast<const f4*>(u.p + e);
      const f4 mv = u.m != nullptr ? *reinterpret_cast<const f4*>(u.m + e) : f4{0.f, 0.f, 0.f, 0.f};
      const f4 vv = u.kind != 0 ? *reinterpret_cast<const f4*>(u.v + e) : f4{0.f, 0.f, 0.f, 0.f};
      f4 pc, mc, vc = f4{0.f, 0.f, 0.f, 0.f};
      float chk = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float pe, me, ve = 0.0f;
        if (u.kind == 0) sgd_element(u, uc.first, pv[c], v[c], mv[c], pe, me, chk);
        else adam_element(u, uc.k, pv[c], v[c], mv[c], vv[c], pe, me, ve, chk);
        pc[c] = pe;
        mc[c] = me;
        vc[c] = ve;
      }
      ok = ok && chk == 0.0f;
      *reinterpret_cast<f4*>(u.pn + e) = pc;
      if (u.mn != nullptr) *reinterpret_cast<f4*>(u.mn + e) = mc;
      if (u.kind != 0) *reinterpret_cast<f4*>(u.vn + e) = vc;
      continue;
    }
    if (p.mode == 0) {
      if (p.bias != nullptr) {
        const f4 b = *reinterpret_cast<const f4*>(p.bias + col);
        v = f4{v[0] + b[0], v[1] + b[1], v[2] + b[2], v[3] + b[3]};
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = apply_act(p.act, v[c]);
    } else {
      const f4 y = *reinterpret_cast<const f4*>(p.aux + row * p.ldaux + col);
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = act_grad(p.act, v[c], y[c]);
    }
    f4* dst = reinterpret_cast<f4*>(p.C + row * p.ldc + col);
    if (p.accumulate) {
      const f4 o = *dst;
      v = f4{o[0] + v[0], o[1] + v[1], o[2] + v[2], o[3] + v[3]};
    }
    *dst = v;
  }
  if (upd) update_flag(p.upd, uc, ok);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

hipError_t launch_tiles(const GemmParams& p, bool va, bool vb, bool split, hipStream_t s) {
  if (!p.transA && !p.transB) return launch_layout<false, false>(p, va, vb, split, s);
  if (!p.transA && p.transB) return launch_layout<false, true>(p, va, vb, split, s);
  if (p.transA && !p.transB) return launch_layout<true, false>(p, va, vb, split, s);
  return launch_layout<true, true>(p, va, vb, split, s);
}

}  // namespace

namespace {
// Split-K plan for problems too small to give every CU a 128x128 tile: slices of at least 128 of
// K, enough of them to reach ~256 workgroups, at most 16.
int64_t splitk_slices(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (K < 512 || tiles >= 128) return 1;
  int64_t s = (256 + tiles - 1) / tiles;
  s = std::min<int64_t>(s, 16);
  s = std::min<int64_t>(s, K / 128);
  return std::max<int64_t>(s, 1);
}
int64_t splitk_chunk(int64_t K, int64_t s) {
  const int64_t c = (K + s - 1) / s;
  return ((c + 31) / 32) * 32;  // whole k-tiles of either tile kernel (BK 16 or 32) per slice
}
}  // namespace

int64_t gemm_workspace_floats(int64_t M, int64_t N, int64_t K, bool colsum) {
  if (M <= 0 || N <= 0) return 0;
  int64_t floats = 0;
  const int64_t s = K > 1 ? splitk_slices(M, N, K) : 1;
  if (s > 1) {
    const int64_t slices = (K + splitk_chunk(K, s) - 1) / splitk_chunk(K, s);
    floats = slices * M * N;
  }
  floats = std::max<int64_t>(floats, skinny_workspace_floats(M, N, K));
  if (colsum && K >= 2 && K <= 16)  // small-K kernel: one binary64 partial row per row block
    floats = std::max<int64_t>(floats, 2 * small_k_row_blocks(M, N) * N);
  if (colsum) {
    // the fused path writes ceil(M/BM) * BM/WM binary64 rows (two K groups of 64x64 tiles:
    // ceil(M/64) * 4), at most (M + 255) / 16 for every configuration; the split path's separate
    // pass needs far fewer
    floats = std::max<int64_t>(floats, 2 * ((M + 255) / 16) * N);
  }
  return floats;
}

namespace {
// float4 loads need the contiguous extent, the leading dimension and the base aligned to 4.
void vector_operands(const GemmParams& p, bool& va, bool& vb) {
  const int64_t a_contig = p.transA ? p.M : p.K;
  const int64_t b_contig = p.transB ? p.K : p.N;
  va = a_contig % 4 == 0 && p.lda % 4 == 0 && aligned16(p.A);
  vb = b_contig % 4 == 0 && p.ldb % 4 == 0 && aligned16(p.B);
}
// Whether this GEMM is split along K: problems with too few 128x128 tiles are, unless the
// direct-to-LDS kernel can run them whole on 64x64 tiles (no partials, no reduction pass).
bool use_split(const GemmParams& in, bool have_workspace) {
  if (!have_workspace || in.K <= 1 || splitk_slices(in.M, in.N, in.K) <= 1) return false;
  GemmParams p = in;
  p.kchunk = 0;
  p.partial = nullptr;
  bool va, vb;
  vector_operands(p, va, vb);
  return !(v2_enabled() && v2_choose(p, va, vb) == 64);
}
}  // namespace

hipError_t launch_gemm_core(const GemmParams& in, float* workspace, hipStream_t s);

// Entry point: runs the GEMM and, when p.colsum is set, the column sum of the stored C -- fused
// into the MFMA epilogue when the GEMM is not split along K, otherwise as a separate pass.
hipError_t launch_gemm(const GemmParams& in, float* workspace, hipStream_t s) {
  GemmParams p = in;
  p.colsum_partial = nullptr;
  if (p.mode == 2 && p.M > 0 && p.N > 0 &&
      (p.K <= 1 || use_split(p, workspace != nullptr) || skinny_route(p) != SKINNY_NONE)) {
    // Mode 2 on a route without the tile kernels' epilogue: the plain forward GEMM, then the
    // cotangent pass and (optionally) its column sum.
    GemmParams f = p;
    f.mode = 0;
    f.aux = nullptr;
    f.dz = nullptr;
    f.colsum = nullptr;
    hipError_t e = launch_gemm_core(f, workspace, s);
    if (e != hipSuccess) return e;
    const unsigned blocks = (unsigned)std::min<int64_t>(65536, (p.M * p.N + 255) / 256);
    hipLaunchKernelGGL(gemm_cotangent_pass, dim3(blocks), dim3(256), 0, s, p.C, p.ldc, p.aux,
                       p.dz, p.ldaux, p.M, p.N, p.act);
    if ((e = hipGetLastError()) != hipSuccess || p.colsum == nullptr) return e;
    return launch_colsum(p.dz, p.colsum, p.M, p.N, p.ldaux, 1.0, 0,
                         reinterpret_cast<double*>(workspace), s);
  }
  if (p.colsum == nullptr || p.M <= 0 || p.N <= 0) return launch_gemm_core(p, workspace, s);
  const bool split = use_split(p, workspace != nullptr);
  const SkinnyRoute route = skinny_route(p);
  if (route == SKINNY_SMALL_K && workspace != nullptr) {  // column sum fused into the kernel
    p.colsum_partial = reinterpret_cast<double*>(workspace);
    hipError_t e = launch_gemm_core(p, workspace, s);
    if (e != hipSuccess) return e;
    return launch_colsum_finish(p.colsum_partial, p.colsum, g_colsum_rows, p.N, s);
  }
  if (p.K <= 1 || split || route != SKINNY_NONE) {
    hipError_t e = launch_gemm_core(p, workspace, s);
    if (e != hipSuccess) return e;
    return launch_colsum(p.C, p.colsum, p.M, p.N, p.ldc, 1.0, 0,
                         reinterpret_cast<double*>(workspace), s);
  }
  p.colsum_partial = reinterpret_cast<double*>(workspace);
  hipError_t e = launch_gemm_core(p, workspace, s);
  if (e != hipSuccess) return e;
  return launch_colsum_finish(p.colsum_partial, p.colsum, g_colsum_rows, p.N, s);
}

hipError_t launch_gemm_core(const GemmParams& in, float* workspace, hipStream_t s) {
  GemmParams p = in;
  p.partial = nullptr;
  p.kchunk = 0;
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  const SkinnyRoute route = skinny_route(p);
  if (route != SKINNY_NONE && (route != SKINNY_COL_OUTER || workspace != nullptr))
    return launch_skinny(p, route, workspace, s);
  if (use_split(p, workspace != nullptr)) {
    p.kchunk = splitk_chunk(p.K, splitk_slices(p.M, p.N, p.K));
    const int slices = (int)((p.K + p.kchunk - 1) / p.kchunk);
    p.partial = workspace;
    bool va, vb;
    vector_operands(p, va, vb);
    hipError_t e = launch_tiles(p, va, vb, true, s);
    if (e != hipSuccess) return e;
    return launch_splitk_finish(p, slices, s);
  }
  if (p.K == 1) {
    const int64_t total = p.M * p.N;
    const unsigned blocks = (unsigned)std::min<int64_t>(65536, (total + 255) / 256);
    hipLaunchKernelGGL(gemm_k1_outer, dim3(blocks), dim3(256), 0, s, p);
    return hipGetLastError();
  }
  bool va, vb;
  vector_operands(p, va, vb);
  return launch_tiles(p, va, vb, false, s);
}

hipError_t launch_splitk_finish(const GemmParams& p, int slices, hipStream_t s) {
  const int64_t total = p.M * p.N;
  bool vec = p.N % 4 == 0 && aligned16(p.partial);
  if (p.upd.pn != nullptr) {
    const GemmUpdate& u = p.upd;
    vec = vec && aligned16(u.p) && aligned16(u.pn) && (u.m == nullptr || (aligned16(u.m) && aligned16(u.mn))) &&
          (u.kind == 0 || (aligned16(u.v) && aligned16(u.vn)));
  } else {
    vec = vec && aligned16(p.C) && p.ldc % 4 == 0 && (p.bias == nullptr || aligned16(p.bias)) &&
          (p.mode != 1 || (aligned16(p.aux) && p.ldaux % 4 == 0));
  }
  if (vec) {
    const unsigned blocks = (unsigned)std::min<int64_t>(65536, (total / 4 + 255) / 256);
    hipLaunchKernelGGL(gemm_splitk_reduce4, dim3(blocks), dim3(256), 0, s, p, slices);
  } else {
    const unsigned blocks = (unsigned)std::min<int64_t>(65536, (total + 255) / 256);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(blocks), dim3(256), 0, s, p, slices);
  }
  return hipGetLastError();
}

}  // namespace shk
