// fp32 MFMA GEMM tile kernel for gfx950 (CDNA4): C = op(A) . op(B) with fused epilogues.
//
// This header holds the tile kernel and its launch templates. Each operand layout (NN, NT, TN,
// TT) instantiates them in a translation unit of its own (gemm_nn.hip ... gemm_tt.hip), so the
// heavy instantiations compile in parallel; gemm.hip holds the dispatch, split-K and K == 1.
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
#pragma once
#include "common.h"
#include "kernels.h"
#include "optim_math.h"
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <utility>

namespace shk {

// Partial rows the last fused-column-sum launch on this thread wrote (ceil(M/BM) * BM/WM).
extern thread_local int64_t g_colsum_rows;

// Launches the MFMA tile kernel for one operand layout (instantiated per layout).
//   va / vb: the A / B operand allows float4 loads; split: p.kchunk > 0 (split-K slices).
template <bool TA, bool TB>
hipError_t launch_layout(const GemmParams& p, bool va, bool vb, bool split, hipStream_t s);
extern template hipError_t launch_layout<false, false>(const GemmParams&, bool, bool, bool, hipStream_t);
extern template hipError_t launch_layout<false, true>(const GemmParams&, bool, bool, bool, hipStream_t);
extern template hipError_t launch_layout<true, false>(const GemmParams&, bool, bool, bool, hipStream_t);
extern template hipError_t launch_layout<true, true>(const GemmParams&, bool, bool, bool, hipStream_t);

namespace {

// Compile-time loop: f(std::integral_constant<int, I>) for I in [0, N). Keeps accumulator
// indexing static where a large #pragma unroll body would be left rolled (and the accumulator
// array demoted to scratch memory).
template <int... I, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

template <int BM, int BN, int BK, int WM, int WN>
struct GemmShape {
  static constexpr int WGM = BM / WM;
  static constexpr int WGN = BN / WN;
  static constexpr int NT = WGM * WGN * 64;
  static constexpr int MI = WM / 32;
  static constexpr int NI = WN / 32;
  static constexpr int PA = BM + 4;  // LDS pitch of the A tile (floats)
  static constexpr int PB = BN + 4;
};

// Fused optimizer update of one element from its gradient g (GemmParams::upd): the candidate
// parameter and slots go to pn/mn/vn; returns false if an intermediate failed its check.
struct UpdateCtx {
  Coeffs k;
  bool first;
};
__device__ __forceinline__ UpdateCtx update_ctx(const GemmUpdate& u) {
  const int64_t completed = *u.completed_steps;
  UpdateCtx c;
  c.first = completed == 0;
  c.k = Coeffs{1.0f, 1.0f, 1.0f, true};
  if (u.kind != 0) c.k = adam_coeffs(u, completed + 1);
  return c;
}
__device__ __forceinline__ bool update_element(const GemmUpdate& u, const UpdateCtx& c,
                                               float pv, float g, float mv, float vv, int64_t e) {
  float pc, mc, vc = 0.0f, chk = 0.0f;
  if (u.kind == 0) sgd_element(u, c.first, pv, g, mv, pc, mc, chk);
  else adam_element(u, c.k, pv, g, mv, vv, pc, mc, vc, chk);
  const bool ok = chk == 0.0f;
  u.pn[e] = pc;
  if (u.mn != nullptr) u.mn[e] = mc;
  if (u.kind != 0) u.vn[e] = vc;
  return ok;
}
// Flags a failed update in the program status word (one atomic per wave).
__device__ __forceinline__ void update_flag(const GemmUpdate& u, const UpdateCtx& c, bool ok) {
  const int bad = wave_or(ok ? 0 : 1);
  if (bad && (threadIdx.x & 63) == 0)
    atomicOr(u.status, c.k.ok ? (uint32_t)DEV_NON_FINITE : (uint32_t)DEV_NOT_POSITIVE);
}
__device__ __forceinline__ bool update_scalar(const GemmUpdate& u, const UpdateCtx& c, int64_t e,
                                              float g) {
  const float mv = u.m != nullptr ? u.m[e] : 0.0f;
  const float vv = u.kind != 0 ? u.v[e] : 0.0f;
  return update_element(u, c, u.p[e], g, mv, vv, e);
}

// Loads one BR x BK tile of an operand into registers and stores it into LDS as [k][r].
//   KCONTIG: element (r, k) lives at ptr[r*ld + k]; otherwise at ptr[k*ld + r].
//   VEC: float4 global loads (the contiguous extent and ld are multiples of 4, ptr 16B aligned).
template <int BR, int BK, int NT, int PITCH, bool KCONTIG, bool VEC>
struct TileLoader {
  static constexpr int ELEMS = BR * BK;
  static constexpr int PER_THREAD = VEC ? ELEMS / 4 / NT : ELEMS / NT;
  static_assert(PER_THREAD >= 1, "tile too small for the workgroup");
  static_assert(VEC ? (ELEMS / 4) % NT == 0 : ELEMS % NT == 0, "uneven tile split");
  using Reg = typename std::conditional<VEC, float4, float>::type;
  Reg reg[PER_THREAD];

  __device__ __forceinline__ void load(const float* __restrict__ ptr, int64_t ld, int64_t r0,
                                       int64_t k0, int64_t R, int64_t K) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int c = tid + i * NT;
      if constexpr (VEC) {
        int r, k;
        if constexpr (KCONTIG) { r = c / (BK / 4); k = (c % (BK / 4)) * 4; }
        else { k = c / (BR / 4); r = (c % (BR / 4)) * 4; }
        const int64_t gr = r0 + r, gk = k0 + k;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (gr < R && gk < K) {
          const float* src = KCONTIG ? ptr + gr * ld + gk : ptr + gk * ld + gr;
          v = *reinterpret_cast<const float4*>(src);
        }
        reg[i] = v;
      } else {
        int r, k;
        if constexpr (KCONTIG) { r = c / BK; k = c % BK; }
        else { k = c / BR; r = c % BR; }
        const int64_t gr = r0 + r, gk = k0 + k;
        float v = 0.f;
        if (gr < R && gk < K) v = KCONTIG ? ptr[gr * ld + gk] : ptr[gk * ld + gr];
        reg[i] = v;
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ lds) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int c = tid + i * NT;
      if constexpr (VEC) {
        if constexpr (KCONTIG) {
          const int r = c / (BK / 4), k = (c % (BK / 4)) * 4;
          lds[(k + 0) * PITCH + r] = reg[i].x;
          lds[(k + 1) * PITCH + r] = reg[i].y;
          lds[(k + 2) * PITCH + r] = reg[i].z;
          lds[(k + 3) * PITCH + r] = reg[i].w;
        } else {
          const int k = c / (BR / 4), r = (c % (BR / 4)) * 4;
          *reinterpret_cast<float4*>(lds + k * PITCH + r) = reg[i];
        }
      } else {
        int r, k;
        if constexpr (KCONTIG) { r = c / BK; k = c % BK; }
        else { k = c / BR; r = c % BR; }
        lds[k * PITCH + r] = reg[i];
      }
    }
  }
};

// Maps the linear workgroup id to an output tile: XCD-contiguous, then grouped along M.
__device__ __forceinline__ void tile_of(int id, int tilesM, int tilesN, int& tm, int& tn) {
  const int total = tilesM * tilesN;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  constexpr int GROUP = 8;
  const int per_group = GROUP * tilesN;
  const int g = id / per_group;
  const int first = g * GROUP;
  const int gsize = min(tilesM - first, GROUP);
  const int in_group = id - g * per_group;
  tm = first + in_group % gsize;
  tn = in_group / gsize;
}

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VA, bool VB, int MINW = 1>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
__attribute__((amdgpu_waves_per_eu(MINW)))
gemm_f32_mfma(GemmParams p) {
  using S = GemmShape<BM, BN, BK, WM, WN>;
  constexpr int NT = S::NT, MI = S::MI, NI = S::NI, PA = S::PA, PB = S::PB;
  __shared__ __attribute__((aligned(16))) float As[2][BK * PA];
  __shared__ __attribute__((aligned(16))) float Bs[2][BK * PB];

  const int tilesM = (int)((p.M + BM - 1) / BM), tilesN = (int)((p.N + BN - 1) / BN);
  int tm, tn;
  tile_of(blockIdx.x, tilesM, tilesN, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / S::WGN, wn = wave % S::WGN;
  const int l32 = lane & 31, half = lane >> 5;

  // A tile: rows m, K-contiguous when A is [M,K] (transA = 0).
  TileLoader<BM, BK, NT, PA, !TA, VA> la;
  // B tile: rows n, K-contiguous when B is stored [N,K] (transB = 1).
  TileLoader<BN, BK, NT, PB, TB, VB> lb;

  floatx16 acc[MI][NI];
  static_for<MI>([&](auto i) {
    static_for<NI>([&](auto j) {
      static_for<16>([&](auto r) { acc[i][j][decltype(r)::value] = 0.f; });
    });
  });

  // K slice of this block row (the whole of K unless split-K is active)
  const int64_t k_begin = p.kchunk > 0 ? (int64_t)blockIdx.y * p.kchunk : 0;
  const int64_t k_end = p.kchunk > 0 ? min(p.K, k_begin + p.kchunk) : p.K;
  const int nk = k_end > k_begin ? (int)((k_end - k_begin + BK - 1) / BK) : 0;
  if (nk > 0) {
    la.load(p.A, p.lda, m0, k_begin, p.M, k_end);
    lb.load(p.B, p.ldb, n0, k_begin, p.N, k_end);
    la.store(As[0]);
    lb.store(Bs[0]);
    __syncthreads();
  }
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(p.A, p.lda, m0, k_begin + (int64_t)(kt + 1) * BK, p.M, k_end);
      lb.load(p.B, p.ldb, n0, k_begin + (int64_t)(kt + 1) * BK, p.N, k_end);
    }
    const float* a_s = As[cur] + wm * (MI * 32) + l32 + half * PA;
    const float* b_s = Bs[cur] + wn * (NI * 32) + l32 + half * PB;
    // Operand fragments are double-buffered in registers: the LDS reads for k-step s+1 are
    // issued before the MFMAs of step s, so their latency hides behind the matrix pipe.
    float a[2][MI], b[2][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i) a[0][i] = a_s[i * 32];
#pragma unroll
    for (int j = 0; j < NI; ++j) b[0][j] = b_s[j * 32];
#pragma unroll
    for (int st = 0; st < BK / 2; ++st) {
      const int c = st & 1;
      if (st + 1 < BK / 2) {
#pragma unroll
        for (int i = 0; i < MI; ++i) a[c ^ 1][i] = a_s[(2 * st + 2) * PA + i * 32];
#pragma unroll
        for (int j = 0; j < NI; ++j) b[c ^ 1][j] = b_s[(2 * st + 2) * PB + j * 32];
      }
      // keep the next fragment's reads ahead of this step's MFMAs (the default scheduler sinks
      // them below to save registers, which exposes the LDS latency again)
      __builtin_amdgcn_sched_barrier(0);
      static_for<MI>([&](auto i) {
        static_for<NI>([&](auto j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[c][i], b[c][j], acc[i][j], 0, 0, 0);
        });
      });
    }
    if (more) {
      la.store(As[cur ^ 1]);
      lb.store(Bs[cur ^ 1]);
    }
    __syncthreads();
  }

  // Epilogue. Accumulator r of a 32x32 block holds row (r/4)*8 + (lane/32)*4 + r%4,
  // column lane%32 of that block. Each block is written from one base pointer with
  // compile-time row offsets, keeping few address registers live.
  if (p.partial != nullptr) {
    // split-K: raw partial sums, reduced (and given the epilogue) by gemm_splitk_reduce
    float* part = p.partial + (int64_t)blockIdx.y * p.M * p.N;
    static_for<NI>([&](auto j) {
      const int64_t col = n0 + wn * (NI * 32) + j * 32 + l32;
      static_for<MI>([&](auto i) {
        const int64_t row0 = m0 + wm * (MI * 32) + i * 32 + half * 4;
        static_for<16>([&](auto r) {
          constexpr int R = decltype(r)::value;
          constexpr int off = (R >> 2) * 8 + (R & 3);
          if (col < p.N && row0 + off < p.M) part[(row0 + off) * p.N + col] = acc[i][j][R];
        });
      });
    });
    return;
  }
  if (p.upd.pn != nullptr) {
    // fused optimizer: per group of four rows, load the current parameters (and slots) of this
    // lane first, then compute and store the candidates
    const GemmUpdate& u = p.upd;
    const UpdateCtx uc = update_ctx(u);
    bool ok = uc.k.ok;
    static_for<NI>([&](auto j) {
      const int64_t col = n0 + wn * (NI * 32) + j * 32 + l32;
      const bool col_ok = col < p.N;
      static_for<MI>([&](auto i) {
        const int64_t row0 = m0 + wm * (MI * 32) + i * 32 + half * 4;
        const int64_t e0 = row0 * p.N + col;
        // four rows at a time: loads of a group are issued together, few registers live
        static_for<4>([&](auto q) {
          constexpr int Q = decltype(q)::value;
          float pv[4], mv[4], vv[4];
          static_for<4>([&](auto r) {
            constexpr int R = decltype(r)::value;
            constexpr int off = Q * 8 + R;
            pv[R] = 0.0f; mv[R] = 0.0f; vv[R] = 0.0f;
            if (col_ok && row0 + off < p.M) {
              pv[R] = u.p[e0 + off * p.N];
              if (u.m != nullptr) mv[R] = u.m[e0 + off * p.N];
              if (u.kind != 0) vv[R] = u.v[e0 + off * p.N];
            }
          });
          static_for<4>([&](auto r) {
            constexpr int R = decltype(r)::value;
            constexpr int off = Q * 8 + R;
            if (col_ok && row0 + off < p.M)
              ok &= update_element(u, uc, pv[R], acc[i][j][Q * 4 + R], mv[R], vv[R], e0 + off * p.N);
          });
        });
        __builtin_amdgcn_sched_barrier(0);
      });
    });
    update_flag(u, uc, ok);
    return;
  }
  static_for<NI>([&](auto j) {
    const int64_t col = n0 + wn * (NI * 32) + j * 32 + l32;
    const bool col_ok = col < p.N;
    const float bias = (p.bias != nullptr && col_ok) ? p.bias[col] : 0.f;
    double csum = 0.0;  // fused column sum of this lane's stored values
    static_for<MI>([&](auto i) {
      const int64_t row0 = m0 + wm * (MI * 32) + i * 32 + half * 4;
      float* cptr = p.C + row0 * p.ldc + col;
      const float* aptr = p.mode != 0 ? p.aux + row0 * p.ldaux + col : nullptr;
      static_for<16>([&](auto r) {
        constexpr int R = decltype(r)::value;
        constexpr int off = (R >> 2) * 8 + (R & 3);
        if (col_ok && row0 + off < p.M) {
          float v = acc[i][j][R];
          if (p.mode != 1) {
            if (p.bias != nullptr) v = v + bias;
            v = apply_act(p.act, v);
          } else {
            v = act_grad(p.act, v, aptr[off * p.ldaux]);
          }
          float* dst = cptr + off * p.ldc;
          if (p.accumulate) v = *dst + v;
          *dst = v;
          if (p.mode == 2) {  // the activation input's cotangent from dY (aux) and the output
            v = act_grad(p.act, aptr[off * p.ldaux], v);
            p.dz[(row0 + off) * p.ldaux + col] = v;
          }
          csum += (double)v;
        }
      });
      __builtin_amdgcn_sched_barrier(0);
    });
    if (p.colsum_partial != nullptr) {
      // lanes l and l+32 hold the same column (different rows): one partial row per wave
      csum += __shfl_xor(csum, 32, 64);
      if (half == 0 && col_ok)
        p.colsum_partial[((int64_t)tm * S::WGM + wm) * p.N + col] = csum;
    }
  });
}

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB,
          int MINW = (BM / WM) * (BN / WN) >= 8 ? 2 : 1>
hipError_t launch_cfg(const GemmParams& p, bool va, bool vb, hipStream_t s) {
  using S = GemmShape<BM, BN, BK, WM, WN>;
  g_colsum_rows = ((p.M + BM - 1) / BM) * (BM / WM);
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const int64_t splits = p.kchunk > 0 ? (p.K + p.kchunk - 1) / p.kchunk : 1;
  dim3 grid((unsigned)tiles, (unsigned)splits), block(S::NT);
  if (va && vb)
    hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, TA, TB, true, true, MINW>), grid, block, 0, s, p);
  else if (va)
    hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, TA, TB, true, false, MINW>), grid, block, 0, s, p);
  else if (vb)
    hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, TA, TB, false, true, MINW>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WM, WN, TA, TB, false, false, MINW>), grid, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace
}  // namespace shk
