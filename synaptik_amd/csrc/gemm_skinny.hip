// Skinny GEMMs for gfx950: C = op(A) . op(B) when one of M, N, K is at most 16.
//
// A classifier head (N = number of classes), its weight gradient (M = classes), the input
// gradient through it (K = classes), a regression head (N = 1) and batch-1 inference (M = 1) are
// all GEMMs with one tiny extent. On 64x64 / 128x128 MFMA tiles at least 7/8 of every tile is
// padding, and the split-K needed to occupy the chip adds a reduction pass; these shapes are
// bandwidth-bound on the wide operand instead. Three kernels, each reading the wide operand once
// along its contiguous axis:
//   * gemm_small_k (2 <= K <= 16): every output is K fused multiply-adds. A thread owns four
//     adjacent columns, keeps their K x 4 B values in registers and walks rows.
//   * gemm_row_dot (narrow output extent J <= 16, wide operand K-contiguous): one wave per wide
//     row, lanes split K (16-byte loads), J accumulators per lane, a butterfly over the wave,
//     and lane j stores output j with the GEMM epilogue.
//   * gemm_col_outer (J <= 16, wide operand [K, cols] with cols contiguous): a thread owns
//     four columns and accumulates J x 4 outer-product terms over a panel of K; panels write
//     binary32 partials that the split-K reduction sums in panel order and finishes with the
//     epilogue.
// The narrow operand is read with a handful of distinct addresses per wave and instruction
// (broadcast from the cache), so its layout does not matter. Narrow extents are compiled in
// buckets of 1, 2, 4, 8 and 16 so that every load is unconditional and issues back to back. The epilogue (bias + activation, activation gradient, accumulation,
// fused optimizer update) is the MFMA kernels' per-element one. Reduction orders differ from the
// MFMA kernels' (fixed and run-to-run identical, within the same reassociation allowance).
#include "gemm_skinny.h"
#include "gemm_tile.h"

namespace shk {
namespace {

constexpr int SK_J = 16;  // largest narrow extent

__device__ __forceinline__ bool epilogue_store(const GemmParams& p, const UpdateCtx& uc,
                                               int64_t row, int64_t col, float v) {
  if (p.upd.pn != nullptr) return update_scalar(p.upd, uc, row * p.N + col, v);
  if (p.mode == 0) {
    if (p.bias != nullptr) v = v + p.bias[col];
    v = apply_act(p.act, v);
  } else {
    v = act_grad(p.act, v, p.aux[row * p.ldaux + col]);
  }
  float* dst = p.C + row * p.ldc + col;
  if (p.accumulate) v = *dst + v;
  *dst = v;
  return true;
}

__device__ __forceinline__ UpdateCtx begin_update(const GemmParams& p, bool& ok) {
  UpdateCtx uc{};
  ok = true;
  if (p.upd.pn != nullptr) {
    uc = update_ctx(p.upd);
    ok = uc.k.ok;
  }
  return uc;
}

// Four consecutive outputs (row, col..col+3) through the epilogue with 16-byte accesses (no
// fused update; N, ldc, ldaux multiples of 4 and C, bias, aux 16-byte aligned). `y` is the
// activation output row segment for mode 1 (loaded by the caller); acc becomes the stored values.
__device__ __forceinline__ void epilogue_store4(const GemmParams& p, int64_t row, int64_t col,
                                                float (&v)[4], const float4& y) {
  if (p.mode == 0) {
    if (p.bias != nullptr) {
      const float4 b = *reinterpret_cast<const float4*>(p.bias + col);
      v[0] = v[0] + b.x; v[1] = v[1] + b.y; v[2] = v[2] + b.z; v[3] = v[3] + b.w;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = apply_act(p.act, v[c]);
  } else {
    v[0] = act_grad(p.act, v[0], y.x); v[1] = act_grad(p.act, v[1], y.y);
    v[2] = act_grad(p.act, v[2], y.z); v[3] = act_grad(p.act, v[3], y.w);
  }
  float4* dst = reinterpret_cast<float4*>(p.C + row * p.ldc + col);
  if (p.accumulate) {
    const float4 o = *dst;
    v[0] = o.x + v[0]; v[1] = o.y + v[1]; v[2] = o.z + v[2]; v[3] = o.w + v[3];
  }
  *dst = make_float4(v[0], v[1], v[2], v[3]);
}

// ---- 2 <= K <= KB ----
// Block x covers 256 columns (lane owns 4); wave w of block row y takes rows y*4 + w + i*S,
// S = gridDim.y * 4, four at a time with all their operand loads issued first. Loads are
// unconditional (indices clamped into range); only terms k < K enter the sum, in order
// k = 0, 1, ... (fmaf). With p.colsum_partial set, the block also sums the stored values of its
// rows per column (binary64; waves added in order through LDS) into colsum_partial[y][N].
//
// CPL is the columns per lane: 4 (a block covers 256 columns, 16-byte accesses when aligned) or,
// for narrow outputs (N <= SMALL_K_NARROW_N), 1 (a block covers 64 columns, every lane of a wave
// has a column of its own, so an expensive epilogue -- the binary64 activation -- is spread over
// four times the lanes). Each output's sum, its epilogue and the blocks' rows (hence the
// column-sum partials) do not depend on CPL: both give identical results.
constexpr int SK_RB = 4;  // rows per wave batch; SK_RB * 16 <= 64 lanes hold a batch's A values
constexpr int64_t SMALL_K_NARROW_N = 128;
// Rows per wave batch: four for 256-column blocks (four columns per lane), one for the narrow
// form (one column per lane), whose outputs are few: one row per wave gives the epilogue's
// per-element work (a binary64 tanh, say) four times the waves instead of a serial loop.
template <int CPL>
constexpr int small_k_rb() { return CPL == 1 ? 1 : SK_RB; }
template <int KB, int CPL>
__global__ void __launch_bounds__(256) gemm_small_k(GemmParams p, int vec_b, int vec_io) {
  constexpr int RB = small_k_rb<CPL>();
  __shared__ double csum[4][64 * CPL];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c0 = ((int64_t)blockIdx.x * 64 + lane) * CPL;
  bool ok;
  const UpdateCtx uc = begin_update(p, ok);
  const int K = (int)p.K;
  const bool want_sum = p.colsum_partial != nullptr;
  double cs[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) cs[c] = 0.0;
  // Every lane runs the row loop, also lanes whose columns lie beyond N (their operand reads
  // are clamped into range and they store nothing): the A values of a batch are loaded by
  // lanes 0 .. RB*KB-1 and read back from them with v_readlane.
  {
    float b[KB][CPL];
    const bool full = c0 + 3 < p.N;
    const bool v4 = CPL == 4 && vec_io && full;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const int64_t kk = k < K ? k : K - 1;
      if (CPL == 4 && vec_b && full) {
        const float4 t = *reinterpret_cast<const float4*>(p.B + kk * p.ldb + c0);
        b[k][0] = t.x; b[k][1 % CPL] = t.y; b[k][2 % CPL] = t.z; b[k][3 % CPL] = t.w;
      } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int64_t col = min(c0 + c, p.N - 1);
          b[k][c] = p.transB ? p.B[col * p.ldb + kk] : p.B[kk * p.ldb + col];
        }
      }
    }
    const int64_t S = (int64_t)gridDim.y * 4;
    for (int64_t r0 = (int64_t)blockIdx.y * 4 + w; r0 < p.M; r0 += S * RB) {
      // The batch's RB x KB A values: lane i*KB + k loads A(row i, k) (one load for the
      // wave), then every lane reads them back from those lanes (v_readlane into SGPRs).
      float a[RB][KB];
      float4 y[RB];
      {
        const int i = lane / KB, k = lane - (lane / KB) * KB;
        const int64_t r = min(r0 + (int64_t)min(i, RB - 1) * S, p.M - 1);
        const int64_t kk = k < K ? k : K - 1;
        const float mine = p.transA ? p.A[kk * p.lda + r] : p.A[r * p.lda + kk];
#pragma unroll
        for (int ii = 0; ii < RB; ++ii)
#pragma unroll
          for (int q = 0; q < KB; ++q)
            a[ii][q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), ii * KB + q));
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int64_t r = min(r0 + i * S, p.M - 1);
        y[i] = (v4 && p.mode == 1) ? *reinterpret_cast<const float4*>(p.aux + r * p.ldaux + c0)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int64_t r = r0 + i * S;
        if (r >= p.M) break;
        float acc[4];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          // from +0, as the reference's sum starts (CpuMatmulReferenceKernel.java:34-119): a
          // first product of -0 must not leave the result -0
          float sum = fmaf(a[i][0], b[0][c], 0.0f);
#pragma unroll
          for (int k = 1; k < KB; ++k) {
            const float t = fmaf(a[i][k], b[k][c], sum);
            sum = k < K ? t : sum;
          }
          acc[c] = sum;
        }
        if (v4) {
          epilogue_store4(p, r, c0, acc, y[i]);
          if (want_sum) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) cs[c] += (double)acc[c];
          }
        } else {
#pragma unroll
          for (int c = 0; c < CPL; ++c) {
            if (c0 + c < p.N) {
              ok &= epilogue_store(p, uc, r, c0 + c, acc[c]);
              if (want_sum) cs[c] += (double)p.C[r * p.ldc + c0 + c];
            }
          }
        }
      }
    }
  }
  if (want_sum) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) csum[w][lane * CPL + c] = cs[c];
    __syncthreads();
    const int64_t col = (int64_t)blockIdx.x * 64 * CPL + threadIdx.x;
    if (threadIdx.x < 64 * CPL && col < p.N)
      p.colsum_partial[(int64_t)blockIdx.y * p.N + col] =
          ((csum[0][threadIdx.x] + csum[1][threadIdx.x]) + csum[2][threadIdx.x]) +
          csum[3][threadIdx.x];
  }
  if (p.upd.pn != nullptr) update_flag(p.upd, uc, ok);
}

// ---- row dot: D[r, j] = sum_k X[r*ldx + k] * Y(j, k), Y(j, k) = Y[j*ysj + k*ysk] ----
// Output (r, j) is C element (r, j), or (j, r) when swap.
struct RowDot {
  const float* X;
  const float* Y;
  int64_t R, K, ldx, ysj, ysk;
  int J, swap, vec;  // vec: X rows and Y(j, .) rows allow 16-byte loads along k
};

// One wave per wide row, lanes over k; JB >= J accumulators (rows j >= J of Y are read clamped
// to J - 1 and their sums dropped), then a butterfly over the wave.
template <int JB>
__global__ void __launch_bounds__(256) gemm_row_dot(GemmParams p, RowDot d) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  bool ok;
  const UpdateCtx uc = begin_update(p, ok);
  if (r < d.R) {
    float acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[j] = 0.0f;
    const float* x = d.X + r * d.ldx;
    if (d.vec) {
#pragma unroll(JB <= 8 ? 4 : 2)
      for (int64_t k = 4 * lane; k < d.K; k += 256) {
        const float4 xv = *reinterpret_cast<const float4*>(x + k);
        float4 yv[JB];
#pragma unroll
        for (int j = 0; j < JB; ++j)
          yv[j] = *reinterpret_cast<const float4*>(d.Y + (j < d.J ? j : d.J - 1) * d.ysj + k);
#pragma unroll
        for (int j = 0; j < JB; ++j) {
          acc[j] = fmaf(xv.x, yv[j].x, acc[j]);
          acc[j] = fmaf(xv.y, yv[j].y, acc[j]);
          acc[j] = fmaf(xv.z, yv[j].z, acc[j]);
          acc[j] = fmaf(xv.w, yv[j].w, acc[j]);
        }
      }
    } else {
#pragma unroll 2
      for (int64_t k = lane; k < d.K; k += 64) {
        const float xv = x[k];
        float yv[JB];
#pragma unroll
        for (int j = 0; j < JB; ++j) yv[j] = d.Y[(j < d.J ? j : d.J - 1) * d.ysj + k * d.ysk];
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[j] = fmaf(xv, yv[j], acc[j]);
      }
    }
    // Transpose-reduce: at offset 32, 16, ... each lane keeps the half of its values that its
    // lane bit selects and adds the partner's copy of that half, so JB values shrink to one
    // in log2(JB) rounds (JB - 1 shuffles); butterflies over the remaining offsets finish the
    // sum. Lane l then holds output j = l >> (6 - log2 JB) (l's top bits, most significant
    // round first).
    constexpr int LG = JB == 1 ? 0 : JB == 2 ? 1 : JB == 4 ? 2 : JB == 8 ? 3 : 4;
    static_for<LG>([&](auto round) {
      constexpr int R = decltype(round)::value;
      constexpr int H = JB >> (R + 1);  // values kept after this round
      const int off = 32 >> R;
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
    const int j = lane >> (6 - LG);
    if ((lane & ((64 >> LG) - 1)) == 0 && j < d.J)
      ok &= d.swap ? epilogue_store(p, uc, j, r, acc[0]) : epilogue_store(p, uc, r, j, acc[0]);
  }
  if (p.upd.pn != nullptr) update_flag(p.upd, uc, ok);
}

// ---- column outer: D[j, col] = sum_k U(k, j) * W[k*ldw + col] over panels of K ----
// Block (x, y) covers 64 columns and the K panel [y*kchunk, min(K, (y+1)*kchunk)): thread t owns
// the four columns 4 (t & 15) .. +3 and the rows k = k0 + (t >> 4) + 16 i. The 16 row phases
// are added in phase order through LDS and the panel sum for output (j, col) -- C element
// (j, col), or (col, j) when swap -- goes to partial[y][M][N].
struct ColOuter {
  const float* W;
  const float* U;
  int64_t cols, K, ldw, usk, usj, kchunk;
  int J, swap, vec;  // vec: W rows allow 16-byte loads
};

template <int JB>
__global__ void __launch_bounds__(256) gemm_col_outer(GemmParams p, ColOuter d) {
  __shared__ float red[16][JB][64];
  const int cg = threadIdx.x & 15, kr = threadIdx.x >> 4;
  const int64_t cbase = (int64_t)blockIdx.x * 64;
  const int64_t c0 = cbase + cg * 4;
  const int64_t k0 = (int64_t)blockIdx.y * d.kchunk;
  const int64_t k1 = min(d.K, k0 + d.kchunk);
  float acc[JB][4];
#pragma unroll
  for (int j = 0; j < JB; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[j][c] = 0.0f;
  const bool full = d.vec && c0 + 3 < d.cols;
#pragma unroll 2
  for (int64_t k = k0 + kr; k < k1; k += 16) {
    float wv[4];
    if (full) {
      const float4 t = *reinterpret_cast<const float4*>(d.W + k * d.ldw + c0);
      wv[0] = t.x; wv[1] = t.y; wv[2] = t.z; wv[3] = t.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) wv[c] = d.W[k * d.ldw + min(c0 + c, d.cols - 1)];
    }
    float u[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) u[j] = d.U[k * d.usk + (j < d.J ? j : d.J - 1) * d.usj];
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[j][c] = fmaf(u[j], wv[c], acc[j][c]);
  }
#pragma unroll
  for (int j = 0; j < JB; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) red[kr][j][cg * 4 + c] = acc[j][c];
  __syncthreads();
  float* plane = p.partial + (int64_t)blockIdx.y * p.M * p.N;
  for (int o = threadIdx.x; o < JB * 64; o += 256) {
    const int j = o >> 6, c = o & 63;
    const int64_t col = cbase + c;
    if (j < d.J && col < d.cols) {
      float sum = red[0][j][c];
#pragma unroll
      for (int q = 1; q < 16; ++q) sum = sum + red[q][j][c];
      plane[d.swap ? col * p.N + j : j * p.N + col] = sum;
    }
  }
}

bool al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

bool skinny_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("SHK_HIP_GEMM_SKINNY");
    return !(e != nullptr && e[0] == '0');
  }();
  return on;
}

int64_t small_k_row_blocks(int64_t M, int64_t N) {
  const int64_t colblocks = (N + 255) / 256;
  const int64_t rb = N <= SMALL_K_NARROW_N ? small_k_rb<1>() : small_k_rb<4>();
  const int64_t rowgroups = (M + 4 * rb - 1) / (4 * rb);  // one row batch per wave
  const int64_t y = std::min<int64_t>(rowgroups, (1024 + colblocks - 1) / colblocks);
  return std::max<int64_t>(1, std::min<int64_t>(y, SMALL_K_MAX_ROW_BLOCKS));
}

int64_t skinny_outer_slices(int64_t cols, int64_t K) {
  const int64_t colblocks = (cols + 63) / 64;
  int64_t s = (512 + colblocks - 1) / colblocks;
  s = std::min<int64_t>(s, (K + 63) / 64);  // at least four rows per thread and panel
  return std::max<int64_t>(1, std::min<int64_t>(s, 32));
}

SkinnyRoute skinny_route(const GemmParams& p) {
  if (!skinny_enabled() || p.M <= 0 || p.N <= 0) return SKINNY_NONE;
  if (p.K >= 2 && p.K <= SK_J) return SKINNY_SMALL_K;
  if (p.K <= SK_J) return SKINNY_NONE;
  if (p.N <= SK_J) return p.transA ? SKINNY_COL_OUTER : SKINNY_ROW_DOT;  // wide operand: A
  if (p.M <= SK_J) return p.transB ? SKINNY_ROW_DOT : SKINNY_COL_OUTER;  // wide operand: B
  return SKINNY_NONE;
}

int64_t skinny_workspace_floats(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= SK_J) return 0;
  int64_t f = 0;
  if (N <= SK_J) f = std::max(f, skinny_outer_slices(M, K) * M * N);
  if (M <= SK_J) f = std::max(f, skinny_outer_slices(N, K) * M * N);
  return f;
}

namespace {
// Smallest compiled bucket (1, 2, 4, 8, 16) holding n.
int bucket(int64_t n) { return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : n <= 8 ? 8 : 16; }

template <template <int> class L, typename... Args>
hipError_t by_bucket(int b, Args&&... args) {
  switch (b) {
    case 1: return L<1>::run(args...);
    case 2: return L<2>::run(args...);
    case 4: return L<4>::run(args...);
    case 8: return L<8>::run(args...);
    default: return L<16>::run(args...);
  }
}

template <int KB>
struct SmallK {
  static hipError_t run(const GemmParams& p, int vec_b, int vec_io, hipStream_t s) {
    const int64_t y = small_k_row_blocks(p.M, p.N);
    if (p.N <= SMALL_K_NARROW_N)
      hipLaunchKernelGGL((gemm_small_k<KB, 1>), dim3((unsigned)((p.N + 63) / 64), (unsigned)y),
                         dim3(256), 0, s, p, vec_b, vec_io);
    else
      hipLaunchKernelGGL((gemm_small_k<KB, 4>), dim3((unsigned)((p.N + 255) / 256), (unsigned)y),
                         dim3(256), 0, s, p, vec_b, vec_io);
    g_colsum_rows = y;
    return hipGetLastError();
  }
};
template <int JB>
struct RowDotL {
  static hipError_t run(const GemmParams& p, const RowDot& d, hipStream_t s) {
    hipLaunchKernelGGL((gemm_row_dot<JB>), dim3((unsigned)((d.R + 3) / 4)), dim3(256), 0, s, p, d);
    return hipGetLastError();
  }
};
template <int JB>
struct ColOuterL {
  static hipError_t run(const GemmParams& p, const ColOuter& d, int64_t panels, hipStream_t s) {
    hipLaunchKernelGGL((gemm_col_outer<JB>), dim3((unsigned)((d.cols + 63) / 64), (unsigned)panels),
                       dim3(256), 0, s, p, d);
    return hipGetLastError();
  }
};
}  // namespace

hipError_t launch_skinny(const GemmParams& in, SkinnyRoute route, float* workspace,
                         hipStream_t s) {
  GemmParams p = in;
  p.partial = nullptr;
  p.kchunk = 0;
  if (route == SKINNY_SMALL_K) {
    const int vec_b = !p.transB && p.N % 4 == 0 && p.ldb % 4 == 0 && al16(p.B);
    const int vec_io = p.upd.pn == nullptr && p.N % 4 == 0 && p.ldc % 4 == 0 && al16(p.C) &&
                       (p.mode != 0 || p.bias == nullptr || al16(p.bias)) &&
                       (p.mode != 1 || (p.ldaux % 4 == 0 && al16(p.aux)));
    const int kb = p.K <= 4 ? 4 : p.K <= 8 ? 8 : p.K <= 12 ? 12 : 16;
    switch (kb) {
      case 4: return SmallK<4>::run(p, vec_b, vec_io, s);
      case 8: return SmallK<8>::run(p, vec_b, vec_io, s);
      case 12: return SmallK<12>::run(p, vec_b, vec_io, s);
      default: return SmallK<16>::run(p, vec_b, vec_io, s);
    }
  }
  if (route == SKINNY_ROW_DOT) {
    RowDot d{};
    if (p.N <= SK_J && !p.transA) {  // rows m of A[M,K]; Y = B as (n, k)
      d.X = p.A; d.ldx = p.lda; d.R = p.M; d.J = (int)p.N; d.swap = 0;
      d.Y = p.B;
      d.ysj = p.transB ? p.ldb : 1;
      d.ysk = p.transB ? 1 : p.ldb;
    } else {                         // rows n of B[N,K]; Y = A as (m, k)
      d.X = p.B; d.ldx = p.ldb; d.R = p.N; d.J = (int)p.M; d.swap = 1;
      d.Y = p.A;
      d.ysj = p.transA ? 1 : p.lda;
      d.ysk = p.transA ? p.lda : 1;
    }
    d.K = p.K;
    d.vec = d.K % 4 == 0 && d.ldx % 4 == 0 && al16(d.X) && d.ysk == 1 && d.ysj % 4 == 0 &&
            al16(d.Y);
    return by_bucket<RowDotL>(bucket(d.J), p, d, s);
  }
  // column outer + panel reduction with the epilogue
  ColOuter d{};
  if (p.N <= SK_J && p.transA) {  // wide A stored [K, M]; U = B as (k, n)
    d.W = p.A; d.ldw = p.lda; d.cols = p.M; d.J = (int)p.N; d.swap = 1;
    d.U = p.B;
    d.usk = p.transB ? 1 : p.ldb;
    d.usj = p.transB ? p.ldb : 1;
  } else {                        // wide B stored [K, N]; U = A as (k, m)
    d.W = p.B; d.ldw = p.ldb; d.cols = p.N; d.J = (int)p.M; d.swap = 0;
    d.U = p.A;
    d.usk = p.transA ? p.lda : 1;
    d.usj = p.transA ? 1 : p.lda;
  }
  d.K = p.K;
  d.vec = d.cols % 4 == 0 && d.ldw % 4 == 0 && al16(d.W);
  const int64_t slices = skinny_outer_slices(d.cols, d.K);
  d.kchunk = (d.K + slices - 1) / slices;
  const int64_t panels = (d.K + d.kchunk - 1) / d.kchunk;
  p.partial = workspace;
  p.kchunk = d.kchunk;
  hipError_t e = by_bucket<ColOuterL>(bucket(d.J), p, d, panels, s);
  if (e != hipSuccess) return e;
  return launch_splitk_finish(p, (int)panels, s);
}

}  // namespace shk
