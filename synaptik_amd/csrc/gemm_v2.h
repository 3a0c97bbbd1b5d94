// Direct-to-LDS fp32 MFMA GEMM tile kernel for gfx950: BT x BT output tiles (BT = 128 or 64),
// BK = 32, four waves of (BT/2) x (BT/2), v_mfma_f32_16x16x4_f32, operands moved from HBM straight
// into LDS.
//
// Used when both operands allow 16-byte loads, K and N are multiples of 4 and the problem gives
// enough workgroups (see v2_choose); ragged M / N / K edges are handled by the TAIL variants.
// Every other case runs the register-staged kernel in gemm_tile.h. The epilogues are the same:
// bias + activation, activation gradient, accumulate, the binary64 column-sum partials of a bias
// gradient, and the staged optimizer update of a weight gradient.
//
// Data movement:
//   * global_load_lds_dwordx4: each lane copies 16 bytes from HBM to LDS without passing through
//     VGPRs; one wave instruction fills 1 KB of LDS. The lane -> address assignment inside an
//     instruction is free, which is used to lay the tile out swizzled (gemm_v2_layout.h). Two LDS
//     stages, software-pipelined so that fragment reads overlap MFMAs and each copy has a whole
//     k-tile of MFMA work to land; one barrier per 32-deep k-tile (see the main loop).
//   * K-contiguous operands (A = X[M,K], B = W[N,K]) are kept [row][k] with 16-byte chunks
//     XOR-swizzled across each 256-byte pair of rows, so that one ds_read_b128 per lane fetches
//     four k values of a row and the 64 lanes of a read hit 64 distinct banks.
//   * M/N-contiguous operands (dZ^T, X, W in [K,N]) are kept [k][row] with chunks swizzled by
//     (k / 4) mod 4; fragments are ds_read_b32.
//   * Edges (TAIL): a lane whose 16-byte chunk lies outside the operand (row >= M or N, k >= K)
//     skips its copy and stores zeros into that LDS chunk instead, so no load leaves the operand
//     and the missing products are exact zeros; the epilogue stores only rows < M, columns < N.
// Reduction order: within a 32-deep k-tile, MFMA s of half h takes k = 16h + 4g + s from lane
// group g; the sum over k is a permutation of the straight order, which the matrix cores
// reassociate anyway (the reference contract allows it, foundational-modules.md:423-425).
#pragma once
#include <cstdlib>
#include <type_traits>

#include "gemm_tile.h"
#include "gemm_v2_layout.h"

namespace shk {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int V2_BK = 32, V2_NT = 256;
// MFMAs per scheduling group: side work (fragment reads, copies) is issued between groups. Four
// for 128-wide tiles (spreads it finer than eight: 4096^3 launches about 0.3% shorter, the
// MLP-4096 step 0.3% faster), two for 64-wide tiles (the C3 classifier step about 0.8% faster
// than with four).
constexpr int V2_GROUP = 4, V2_GROUP64 = 2;

template <int BT>
struct V2Cfg {
  static constexpr int NB = BT / 32;      // 16x16 blocks per wave and dimension
  static constexpr int WT = BT / 2;       // wave tile edge
  static constexpr int TILEF = BT * 32;   // floats per operand per stage
  static constexpr int NI = BT / 32;      // copies per thread per operand per k-tile
  static constexpr int CPR = BT / 4;      // 16-byte chunks per k-row of an M/N-contiguous tile
  static constexpr int GS = BT == 64 ? V2_GROUP64 : V2_GROUP;  // MFMAs per group
  static constexpr int NG = 4 * NB * NB / GS;  // MFMA groups per half k-tile
  static constexpr int CPG = 4 * NI / NG;  // copies issued after a group
  static constexpr int ECPR = WT / 4;     // 16-byte chunks per row of the epilogue transpose
};

// Per-lane source offsets (bytes, relative to the tile origin) of the NI 16-byte copies this
// thread issues per operand per k-tile, where they land, and (TAIL) the chunk's coordinates.
template <bool KMAJ, int BT, bool TAIL>
struct V2Loader {
  using Cfg = V2Cfg<BT>;
  uint32_t voff[Cfg::NI];
  int vrow[Cfg::NI], vk[Cfg::NI];  // first row (M/N) and first k of the chunk in the tile
  uint32_t wdst;                   // this wave's byte offset inside a stage (wave-uniform)
  __device__ __forceinline__ void init(int64_t ld) {
    const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3;
    wdst = __builtin_amdgcn_readfirstlane((uint32_t)w * 1024u);
#pragma unroll
    for (int i = 0; i < Cfg::NI; ++i) {
      const int q = (i * 4 + w) * 64 + lane;  // destination chunk of this lane
      if constexpr (KMAJ) {
        const int src = v2_kmaj_src(q), r = src >> 3, c = src & 7;
        voff[i] = (uint32_t)((r * ld + 4 * c) * 4);
        vrow[i] = r;
        vk[i] = 4 * c;
      } else {
        const int src = v2_mnmaj_src(q, Cfg::CPR), k = src / Cfg::CPR, c = src % Cfg::CPR;
        voff[i] = (uint32_t)((k * ld + 4 * c) * 4);
        vrow[i] = 4 * c;
        vk[i] = k;
      }
    }
  }
  // Copy I of this wave for the k-tile whose element (row 0, k 0) is `tile`, into stage `lds`:
  // global_load_lds_dwordx4 with the tile origin in SGPRs, a per-lane 32-bit offset and the LDS
  // destination in M0. Written as inline assembly so that the compiler does not track the copies
  // (it would make every LDS read wait for all copies in flight, including those into the other
  // stage); the kernel waits for them itself (v2_wait_all) before each barrier.
  // TAIL: rows_left / k_left bound the valid part of the tile; other lanes store zeros.
  template <int I>
  __device__ __forceinline__ void issue(const float* tile, float* lds, int rows_left,
                                        int k_left) const {
    const uint32_t dst =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)lds + I * 4096u + wdst;
    // a whole tile row-range and a whole k-tile (uniform) need no per-lane bounds
    if (!TAIL || (rows_left >= BT && k_left >= V2_BK) || (vrow[I] < rows_left && vk[I] < k_left)) {
      asm volatile("global_load_lds_dwordx4 %0, %1"
                   :
                   : "v"(voff[I]), "s"(tile), "{m0}"(dst)
                   : "memory");
    } else {
      const int w = (threadIdx.x >> 6) & 3, lane = threadIdx.x & 63;
      *reinterpret_cast<floatx4*>(lds + (I * 4 + w) * 256 + lane * 4) = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
};

// Fragments of one operand for one half (16 k) of a k-tile: f[b][s] is the value lane
// (MFMA row l16 = lane % 16 of block b; group g = lane / 16) supplies to MFMA s.
//
// K-contiguous operands: block b of the wave's sub-tile is rows 16b .. 16b + 15, and one
// ds_read_b128 per block returns the four k values a lane needs (item b reads block b).
// base[0] / base[1] are the offsets of this lane's chunk (4H + g) in the wave's rows 0..15 /
// 16..31; blocks 2 and 3 repeat them 32 rows (1024 floats) further.
//
// M/N-contiguous operands are stored [k][row], where a 16-byte chunk holds four consecutive rows
// at one k. Their blocks interleave instead: block b is the wave's rows NB r + b (r = 0..15), so
// the NB values a lane needs at one k (row NB l16 + b of every block) are adjacent, and one read
// of NB floats (ds_read_b128 for NB = 4, ds_read_b64 for NB = 2) per k fills f[0..NB)[s] (item s
// reads MFMA step s). base[0] is the offset of (k = 4g, row NB l16); the k-row 16H + 4g + s
// adds (16H + s) * BT (the chunk swizzle depends on (k / 4) mod 4 = g only). The epilogue maps
// the accumulators back through the same interleave (v2_row / v2_col).
template <bool KMAJ, int BT>
struct V2Frag {
  static constexpr int NB = V2Cfg<BT>::NB;
  static constexpr int ITEMS = KMAJ ? NB : 4;  // fragment reads per half
  floatx4 f[NB];
  template <int H, int T>
  __device__ __forceinline__ void load_item(const float* lds, const int* base) {
    if constexpr (KMAJ) {
      f[T] = *reinterpret_cast<const floatx4*>(lds + base[T & 1] + (T >> 1) * 1024);
    } else if constexpr (NB == 4) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(lds + base[0] + (16 * H + T) * BT);
      static_for<4>([&](auto b) { f[decltype(b)::value][T] = v[decltype(b)::value]; });
    } else {
      typedef float floatx2 __attribute__((ext_vector_type(2)));
      const floatx2 v = *reinterpret_cast<const floatx2*>(lds + base[0] + (16 * H + T) * BT);
      f[0][T] = v[0];
      f[1][T] = v[1];
    }
  }
  template <int H>
  __device__ __forceinline__ void load(const float* lds, const int* base) {
    static_for<ITEMS>([&](auto t) { load_item<H, decltype(t)::value>(lds, base); });
  }
};

// Order in which the 2 NB-to-8 fragment reads of a half are issued: by the index of the first
// MFMA that uses them (MFMA n = s NB^2 + i NB + j uses A item (KA ? i : s) and B item
// (KB ? j : s)), A before B on ties; the all-K-contiguous case keeps A0 B0 B1 A1 B2 B3 A2 A3.
template <bool KA, bool KB, int NB>
struct V2ReadOrder {
  static constexpr int IA = KA ? NB : 4, IB = KB ? NB : 4, N = IA + IB;
  int op[8] = {}, idx[8] = {};
  constexpr V2ReadOrder() {
    if (KA && KB && NB == 4) {
      const int o[8] = {0, 1, 1, 0, 1, 1, 0, 0}, b[8] = {0, 0, 1, 1, 2, 3, 2, 3};
      for (int t = 0; t < 8; ++t) { op[t] = o[t]; idx[t] = b[t]; }
      return;
    }
    int ia = 0, ib = 0;
    for (int t = 0; t < N; ++t) {
      const int ua = ia < IA ? (KA ? ia * NB : ia * NB * NB) : 1 << 20;
      const int ub = ib < IB ? (KB ? ib : ib * NB * NB) : 1 << 20;
      if (ua <= ub) { op[t] = 0; idx[t] = ia++; }
      else { op[t] = 1; idx[t] = ib++; }
    }
  }
};

__device__ __forceinline__ void v2_wait_all() {
  // vmcnt(0) and lgkmcnt(0): this wave's LDS copies have landed and its LDS reads returned
  __builtin_amdgcn_s_waitcnt(0x0070);
}
// Workgroup barrier that is also a compiler memory barrier (no LDS access moves across it).
__device__ __forceinline__ void v2_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The tile kernel. KA: A(m, k) is contiguous along k (A stored [M,K]); KB: B(n, k) is contiguous
// along k (B stored [N,K]). KS = 2 splits K inside the workgroup: eight waves in two groups of
// four, group h runs the whole pipeline below on k-tiles [h T, (h + 1) T), T = ceil(k-tiles / 2),
// of the workgroup's K range (all of K, or its split-K slice), with LDS stages of its own (group
// 1's last tile is all zeros when the count is odd: TAIL); both groups stage their partial tiles
// in LDS and share the epilogue, each value the sum group 0 + group 1 (a fixed order), stored as
// the result or, for a slice, as the slice's partial. It gives each SIMD two waves on problems
// with too few tiles for two workgroups per CU, without more partials in HBM or a second launch.
template <bool KA, bool KB, int BT, bool TAIL, int KS>
__global__ void __launch_bounds__(V2_NT * KS) __attribute__((amdgpu_waves_per_eu(2)))
gemm_f32_v2(GemmParams p) {
  using Cfg = V2Cfg<BT>;
  constexpr int NB = Cfg::NB, WT = Cfg::WT, TILEF = Cfg::TILEF, NI = Cfg::NI, NG = Cfg::NG;
  __shared__ __attribute__((aligned(16))) float As0g[KS * TILEF];
  __shared__ __attribute__((aligned(16))) float Bs0g[KS * TILEF];
  __shared__ __attribute__((aligned(16))) float As1g[KS * TILEF];
  __shared__ __attribute__((aligned(16))) float Bs1g[KS * TILEF];
  // wave-uniform (readfirstlane): tile origins derived from it stay in SGPRs
  const int kgroup = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));
  float* const As0 = As0g + kgroup * TILEF;
  float* const Bs0 = Bs0g + kgroup * TILEF;
  float* const As1 = As1g + kgroup * TILEF;
  float* const Bs1 = Bs1g + kgroup * TILEF;

  const int tilesM = (int)((p.M + BT - 1) / BT), tilesN = (int)((p.N + BT - 1) / BT);
  int tm, tn;
  tile_of(blockIdx.x, tilesM, tilesN, tm, tn);
  const int64_t m0 = (int64_t)tm * BT, n0 = (int64_t)tn * BT;
  const int lane = threadIdx.x & 63, wave = (threadIdx.x >> 6) & 3;
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, g = lane >> 4;
  const int rows_a = (int)std::min<int64_t>(BT, p.M - m0);
  const int rows_b = (int)std::min<int64_t>(BT, p.N - n0);

  // operand tile origins at k = 0, and the per-k-tile advance
  // split-K: block row y covers k in [y * kchunk, min(K, (y + 1) * kchunk))
  int64_t k_begin = p.kchunk > 0 ? (int64_t)blockIdx.y * p.kchunk : 0;
  int64_t k_len = p.kchunk > 0 ? std::min<int64_t>(p.kchunk, p.K - k_begin) : p.K;
  int nk = (int)((k_len + V2_BK - 1) / V2_BK);
  if constexpr (KS == 2) {  // the two groups halve the slice [k_begin, k_begin + k_len)
    const int half = (nk + 1) / 2;
    const int64_t len = k_len;
    k_begin += (int64_t)kgroup * half * V2_BK;
    k_len = kgroup == 0 ? std::min<int64_t>(len, (int64_t)half * V2_BK) : len - (int64_t)half * V2_BK;
    nk = half;  // group 1: k_len may end inside (or before) its last tile, which TAIL zero-fills
  }
  const float* a_tile = KA ? p.A + m0 * p.lda + k_begin : p.A + m0 + k_begin * p.lda;
  const float* b_tile = KB ? p.B + n0 * p.ldb + k_begin : p.B + n0 + k_begin * p.ldb;
  const int64_t a_step = KA ? V2_BK : V2_BK * p.lda;
  const int64_t b_step = KB ? V2_BK : V2_BK * p.ldb;
  V2Loader<KA, BT, TAIL> la;
  V2Loader<KB, BT, TAIL> lb;
  la.init(p.lda);
  lb.init(p.ldb);

  // lane-dependent fragment offsets per half (see V2Frag)
  int a_base[2][NB], b_base[2][NB];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      a_base[h][q] = KA ? v2_kmaj_off(wm * WT + 16 * (q & 1) + l16, 4 * h + g)
                        : v2_mnmaj_off(4 * g, wm * WT + NB * l16, Cfg::CPR);
      b_base[h][q] = KB ? v2_kmaj_off(wn * WT + 16 * (q & 1) + l16, 4 * h + g)
                        : v2_mnmaj_off(4 * g, wn * WT + NB * l16, Cfg::CPR);
    }
  }
  // Wave sub-tile row and column of accumulator register R of block (I, J). The MFMA's output
  // lane holds four consecutive rows (4g + R) of one column (l16) of its 16 x 16 block. With a
  // K-contiguous B the operands go into the MFMA swapped (it computes the block's transpose:
  // products and sums are the same), so that a lane holds four consecutive columns of one row
  // instead and the epilogue stages them with one 16-byte LDS write; an M/N-contiguous B already
  // gives a lane NB adjacent columns through its interleaved blocks.
  auto v2_row = [&](int I, int R) {
    if constexpr (KB) return KA ? 16 * I + l16 : NB * l16 + I;
    else return KA ? 16 * I + 4 * g + R : NB * (4 * g + R) + I;
  };
  auto v2_col = [&](int J, int R) {
    if constexpr (KB) return 16 * J + 4 * g + R;
    else return NB * l16 + J;
  };

  floatx4 acc[NB][NB];
  static_for<NB>([&](auto i) {
    static_for<NB>([&](auto j) {
      acc[decltype(i)::value][decltype(j)::value] = floatx4{0.f, 0.f, 0.f, 0.f};
    });
  });

  // 4 NB^2 MFMAs of one half-tile in NG groups of V2_GROUP (MFMA n: s = n / NB^2, block
  // i = (n % NB^2) / NB, j = n % NB, or i and j exchanged for a K-contiguous B); after each group, side(q) issues that group's share of the
  // LDS reads and copies. The scheduling barriers keep this order: reads and copies spread over
  // the MFMA stream instead of stalling it in one place.
  auto mfma_half = [&](const V2Frag<KA, BT>& fa, const V2Frag<KB, BT>& fb, auto side) {
    static_for<NG>([&](auto q) {
      constexpr int Q = decltype(q)::value;
      static_for<Cfg::GS>([&](auto u) {
        constexpr int N = Cfg::GS * Q + decltype(u)::value;
        // (with the operands swapped, consecutive MFMAs share their first operand)
        constexpr int S = N / (NB * NB);
        constexpr int I = KB ? N % NB : (N % (NB * NB)) / NB;
        constexpr int J = KB ? (N % (NB * NB)) / NB : N % NB;
        if constexpr (KB)
          acc[I][J] = __builtin_amdgcn_mfma_f32_16x16x4f32(fb.f[J][S], fa.f[I][S], acc[I][J], 0,
                                                          0, 0);
        else
          acc[I][J] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.f[I][S], fb.f[J][S], acc[I][J], 0,
                                                          0, 0);
      });
      __builtin_amdgcn_sched_barrier(0);
      side(q);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // Fragment reads of half H from stage (As, Bs): read item t in V2ReadOrder (the items the next
  // half's first MFMAs use come first); group q issues items q RPG .. q RPG + RPG - 1.
  constexpr V2ReadOrder<KA, KB, NB> kOrder{};
  constexpr int NREAD = kOrder.N, RPG = (NREAD + NG / 2 - 1) / (NG / 2);
  auto read_item = [&](auto t, V2Frag<KA, BT>& fa, V2Frag<KB, BT>& fb, const float* As,
                       const float* Bs, auto h) {
    constexpr int T = decltype(t)::value, H = decltype(h)::value;
    if constexpr (T < NREAD) {
      if constexpr (kOrder.op[T] == 0) fa.template load_item<H, kOrder.idx[T]>(As, a_base[H]);
      else fb.template load_item<H, kOrder.idx[T]>(Bs, b_base[H]);
    }
  };
  // Copies of a k-tile: item c (c < 2 NI) is operand c % 2, instruction c / 2.
  auto copy_item = [&](auto c, const float* at, const float* bt, float* As, float* Bs, int k_left) {
    constexpr int C = decltype(c)::value;
    if constexpr (C % 2 == 0) la.template issue<C / 2>(at, As, rows_a, k_left);
    else lb.template issue<C / 2>(bt, Bs, rows_b, k_left);
  };
  auto copy_all = [&](const float* at, const float* bt, float* As, float* Bs, int k_left) {
    static_for<2 * NI>([&](auto c) { copy_item(c, at, bt, As, Bs, k_left); });
  };

  // Software pipeline over k-tiles (tile kt lives in stage kt % 2; fa0 / fb0 hold its first-half
  // fragments on entry):
  //   first half: MFMAs with fa0 / fb0 while the second-half fragments load into fa1 / fb1;
  //   wait for this wave's copies and reads, barrier: tile kt+1 has landed everywhere and every
  //   wave has read all of tile kt;
  //   second half: MFMAs with fa1 / fb1 while tile kt+1's first-half fragments load into
  //   fa0 / fb0 (first half of the groups) and tile kt+2 is copied into tile kt's stage (second
  //   half of the groups).
  // Each copy has most of a k-tile of MFMA work to land; no LDS read touches a stage while a
  // copy into it is in flight.
  V2Frag<KA, BT> fa0, fa1;
  V2Frag<KB, BT> fb0, fb1;
  copy_all(a_tile, b_tile, As0, Bs0, (int)k_len);
  if (nk > 1) {
    copy_all(a_tile + a_step, b_tile + b_step, As1, Bs1, (int)(k_len - V2_BK));
    // vmcnt(2 NI) says the first k-tile's copies have landed only when every lane issued all
    // of its copies for both k-tiles: otherwise (lanes that stored zeros) wait for everything
    if (TAIL && !(rows_a == BT && rows_b == BT && k_len >= 2 * V2_BK)) {
      v2_wait_all();
    } else {
      if constexpr (NI == 4) __builtin_amdgcn_s_waitcnt(0x0F78);
      else __builtin_amdgcn_s_waitcnt(0x0F74);
    }
  } else {
    v2_wait_all();
  }
  v2_barrier();
  fa0.template load<0>(As0, a_base[0]);
  fb0.template load<0>(Bs0, b_base[0]);
  auto step = [&](auto cur, int kt) {
    constexpr int CUR = decltype(cur)::value;
    float* Acur = CUR ? As1 : As0;
    float* Bcur = CUR ? Bs1 : Bs0;
    const float* Aoth = CUR ? As0 : As1;
    const float* Both = CUR ? Bs0 : Bs1;
    const bool more = kt + 1 < nk, copy = kt + 2 < nk;
    const float* at = a_tile + (int64_t)(kt + 2) * a_step;
    const float* bt = b_tile + (int64_t)(kt + 2) * b_step;
    const int k_left = (int)(k_len - (int64_t)(kt + 2) * V2_BK);
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(fa0, fb0, [&](auto q) {
      constexpr int Q = decltype(q)::value;
      if constexpr (Q < NG / 2) {
        static_for<RPG>([&](auto r) {
          read_item(std::integral_constant<int, Q * RPG + decltype(r)::value>{}, fa1, fb1,
                    Acur, Bcur, std::integral_constant<int, 1>{});
        });
      }
    });
    if (more) {
      v2_wait_all();
      v2_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(fa1, fb1, [&](auto q) {
      constexpr int Q = decltype(q)::value;
      if constexpr (Q < NG / 2) {
        if (more) {
          static_for<RPG>([&](auto r) {
            read_item(std::integral_constant<int, Q * RPG + decltype(r)::value>{}, fa0, fb0,
                      Aoth, Both, std::integral_constant<int, 0>{});
          });
        }
      } else {
        if (copy) {
          static_for<Cfg::CPG>([&](auto c) {
            copy_item(std::integral_constant<int, (Q - NG / 2) * Cfg::CPG + decltype(c)::value>{},
                      at, bt, Acur, Bcur, k_left);
          });
        }
      }
    });
  };
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    step(std::integral_constant<int, 0>{}, kt);
    step(std::integral_constant<int, 1>{}, kt + 1);
  }
  if (kt < nk) step(std::integral_constant<int, 0>{}, kt);

  // Epilogue. Accumulator r of block (i, j) holds row 16i + 4g + r, column 16j + l16 of the
  // wave's WT x WT sub-tile. Split-K partials are written from that layout directly; otherwise
  // the sub-tile is transposed through this wave's own part of the (now free) LDS stages
  // (row-major, 16-byte chunks XOR-swizzled by row) so that every global access of the epilogue
  // is a 16-byte row segment: lane (q = lane % ECPR, rg = lane / ECPR) owns columns 4q..4q+3 of
  // rows rg + (64 / ECPR) t, and each store instruction covers whole WT-float row segments.
  if (KS == 1 && p.partial != nullptr) {
    // split-K: raw partial sums, reduced (and given the epilogue) by gemm_splitk_reduce
    float* part = p.partial + (int64_t)blockIdx.y * p.M * p.N;
    static_for<NB>([&](auto i) {
      static_for<NB>([&](auto j) {
        constexpr int I = decltype(i)::value, J = decltype(j)::value;
        static_for<4>([&](auto r) {
          constexpr int R = decltype(r)::value;
          const int64_t row = m0 + wm * WT + v2_row(I, R);
          const int64_t col = n0 + wn * WT + v2_col(J, R);
          if (!TAIL || (row < p.M && col < p.N)) part[row * p.N + col] = acc[I][J][R];
        });
      });
    });
    return;
  }
  v2_wait_all();
  v2_barrier();  // every wave has finished reading its fragments: the stages are free
  constexpr int ECPR = Cfg::ECPR, RSTEP = 64 / ECPR, PER_ARRAY = TILEF / (WT * WT);
  const int arr = wave / PER_ARRAY;
  float* stage = (arr == 0 ? As0 : arr == 1 ? Bs0 : arr == 2 ? As1 : Bs1) +
                 (wave % PER_ARRAY) * (WT * WT);
  if constexpr (KB) {
    // the four registers of block (I, J) are columns 16 J + 4g .. + 3 of one row
    static_for<NB>([&](auto i) {
      static_for<NB>([&](auto j) {
        constexpr int I = decltype(i)::value, J = decltype(j)::value;
        const int row = v2_row(I, 0), col = v2_col(J, 0);
        *reinterpret_cast<floatx4*>(stage + row * WT + (((col >> 2) ^ (row % ECPR)) << 2)) =
            acc[I][J];
      });
    });
  } else {
    // the NB columns NB l16 + J (J < NB) of a lane are adjacent: one NB-float store per row
    static_for<NB>([&](auto i) {
      static_for<4>([&](auto r) {
        constexpr int I = decltype(i)::value, R = decltype(r)::value;
        const int row = v2_row(I, R), col = NB * l16;
        float* dst = stage + row * WT + (((col >> 2) ^ (row % ECPR)) << 2) + (col & 3);
        if constexpr (NB == 4) {
          *reinterpret_cast<floatx4*>(dst) =
              floatx4{acc[I][0][R], acc[I][1][R], acc[I][2][R], acc[I][3][R]};
        } else {
          typedef float floatx2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<floatx2*>(dst) = floatx2{acc[I][0][R], acc[I][1][R]};
        }
      });
    });
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are complete
  // KS = 2: each group has staged its partial tile in its own stages; after the barrier group h
  // stores rows [h WT / 2, (h + 1) WT / 2) of every wave tile, each value the sum of the two
  // partial tiles in a fixed order (group 0's + group 1's), so both groups share the epilogue.
  if constexpr (KS == 2) v2_barrier();
  const float* stage0 = (arr == 0 ? As0g : arr == 1 ? Bs0g : arr == 2 ? As1g : Bs1g) +
                        (wave % PER_ARRAY) * (WT * WT);
  const int q = lane % ECPR, rg = lane / ECPR;
  auto tile_row = [&](int t) -> floatx4 {
    const int row = rg + RSTEP * t;
    const int off = row * WT + ((q ^ (row % ECPR)) << 2);
    if constexpr (KS == 1) {
      return *reinterpret_cast<const floatx4*>(stage + off);
    } else {
      const floatx4 v0 = *reinterpret_cast<const floatx4*>(stage0 + off);
      const floatx4 v1 = *reinterpret_cast<const floatx4*>(stage0 + TILEF + off);
      return floatx4{v0[0] + v1[0], v0[1] + v1[1], v0[2] + v1[2], v0[3] + v1[3]};
    }
  };
  static_assert(KS == 1 || (WT / RSTEP) % KS == 0, "row steps split evenly between the groups");
  constexpr int TSTEPS = WT / RSTEP / KS;  // row steps per group
  // row steps per chunk of the update loop (128-wide tiles: 16 row steps per lane; the 64-wide
  // tiles' two measured faster unchunked)
  constexpr int EPI_CH = BT == 128 ? 4 : 1;
  static_assert(TSTEPS % EPI_CH == 0, "whole chunks");
  const int tfirst = kgroup * TSTEPS;
  const int64_t row_e = m0 + wm * WT + rg, col_e = n0 + wn * WT + 4 * q;
  const bool col_ok = !TAIL || col_e < p.N;  // N is a multiple of 4: whole segments
  if constexpr (KS == 2) {
    if (p.partial != nullptr) {
      // split-K slice of a KS = 2 workgroup: the slice's partial sums (group 0's + group 1's),
      // in 16-byte row segments, reduced (and given the epilogue) by gemm_splitk_reduce
      float* part = p.partial + (int64_t)blockIdx.y * p.M * p.N;
      for (int t = tfirst; t < tfirst + TSTEPS; ++t) {
        const int64_t row = row_e + RSTEP * t;
        if (TAIL && (!col_ok || row >= p.M)) continue;
        *reinterpret_cast<floatx4*>(part + row * p.N + col_e) = tile_row(t);
      }
      return;
    }
  }
  // The loops below are compiled once per optimizer kind / (mode, activation, accumulate): a
  // runtime switch inside them would make every LDS read and store wait for the one before.
  if (p.upd.pn != nullptr) {
    const GemmUpdate& u = p.upd;
    const UpdateCtx uc = update_ctx(u);
    bool ok = uc.k.ok;
    float chk = 0.0f;  // NaN once any intermediate of this lane's elements was not finite
    auto update_rows = [&](auto kindc) {
      constexpr bool SGD = decltype(kindc)::value == 0;
      // EPI_CH row steps at a time: every parameter and slot load of the chunk is issued before
      // its first store, so the loads' latencies overlap instead of adding up row after row
      for (int t0 = tfirst; t0 < tfirst + TSTEPS; t0 += EPI_CH) {
        floatx4 pv[EPI_CH], mv[EPI_CH], vv[EPI_CH];
        static_for<EPI_CH>([&](auto ic) {
          constexpr int I = decltype(ic)::value;
          const int64_t row = row_e + RSTEP * (t0 + I);
          const bool in = !TAIL || (col_ok && row < p.M);
          const int64_t e = row * p.N + col_e;
          const floatx4 z = floatx4{0.f, 0.f, 0.f, 0.f};
          pv[I] = in ? *reinterpret_cast<const floatx4*>(u.p + e) : z;
          mv[I] = in && u.m != nullptr ? *reinterpret_cast<const floatx4*>(u.m + e) : z;
          vv[I] = !SGD && in ? *reinterpret_cast<const floatx4*>(u.v + e) : z;
        });
        static_for<EPI_CH>([&](auto ic) {
          constexpr int I = decltype(ic)::value;
          const int64_t row = row_e + RSTEP * (t0 + I);
          if (TAIL && (!col_ok || row >= p.M)) return;
          const int64_t e = row * p.N + col_e;
          const floatx4 gv = tile_row(t0 + I);
          floatx4 pc, mc, vc = floatx4{0.f, 0.f, 0.f, 0.f};
          static_for<4>([&](auto c) {
            constexpr int C = decltype(c)::value;
            float pe, me, ve = 0.0f;
            if constexpr (SGD) sgd_element(u, uc.first, pv[I][C], gv[C], mv[I][C], pe, me, chk);
            else adam_element(u, uc.k, pv[I][C], gv[C], mv[I][C], vv[I][C], pe, me, ve, chk);
            pc[C] = pe;
            mc[C] = me;
            vc[C] = ve;
          });
          *reinterpret_cast<floatx4*>(u.pn + e) = pc;
          if (u.mn != nullptr) *reinterpret_cast<floatx4*>(u.mn + e) = mc;
          if constexpr (!SGD) *reinterpret_cast<floatx4*>(u.vn + e) = vc;
        });
      }
    };
    if (u.kind == 0) update_rows(std::integral_constant<int, 0>{});
    else update_rows(std::integral_constant<int, 1>{});
    update_flag(u, uc, ok && chk == 0.0f);
    return;
  }
  const bool has_bias = p.bias != nullptr;
  floatx4 bias = floatx4{0.f, 0.f, 0.f, 0.f};
  if (has_bias && col_ok) bias = *reinterpret_cast<const floatx4*>(p.bias + col_e);
  double cs[4] = {0.0, 0.0, 0.0, 0.0};  // fused column sums of this lane's stored values
  auto store_rows = [&](auto modec, auto actc, auto accc) {
    constexpr int MODE = decltype(modec)::value, ACT = decltype(actc)::value;
    constexpr bool ACC = decltype(accc)::value;
    // Modes 1 and 2 read one aux row segment per row step (the activation output, or dY): the
    // loads of a chunk of SCH row steps are issued before the chunk's first store, so their
    // latencies overlap instead of adding up row step after row step (the accumulators are
    // staged in LDS by now, which frees their registers; 16 row steps at once would spill).
    constexpr int SCH = TSTEPS < 8 ? TSTEPS : 8;
    static_assert(TSTEPS % SCH == 0, "whole chunks");
    for (int t0 = tfirst; t0 < tfirst + TSTEPS; t0 += SCH) {
      floatx4 ya[SCH];
      if constexpr (MODE != 0) {
        static_for<SCH>([&](auto ic) {
          constexpr int I = decltype(ic)::value;
          const int64_t row = row_e + RSTEP * (t0 + I);
          ya[I] = (!TAIL || (col_ok && row < p.M))
                      ? *reinterpret_cast<const floatx4*>(p.aux + row * p.ldaux + col_e)
                      : floatx4{0.f, 0.f, 0.f, 0.f};
        });
      }
      static_for<SCH>([&](auto ic) {
        constexpr int I = decltype(ic)::value;
        const int t = t0 + I;
        const int64_t row = row_e + RSTEP * t;
        if (TAIL && (!col_ok || row >= p.M)) return;
        floatx4 v = tile_row(t);
        if constexpr (MODE != 1) {
          if (has_bias) v = floatx4{v[0] + bias[0], v[1] + bias[1], v[2] + bias[2], v[3] + bias[3]};
          static_for<4>([&](auto c) { v[decltype(c)::value] = apply_act(ACT, v[decltype(c)::value]); });
        } else {
          const floatx4 y = ya[I];
          static_for<4>([&](auto c) {
            constexpr int C = decltype(c)::value;
            v[C] = act_grad(ACT, v[C], y[C]);
          });
        }
        floatx4* dst = reinterpret_cast<floatx4*>(p.C + row * p.ldc + col_e);
        if constexpr (ACC) {
          const floatx4 o = *dst;
          v = floatx4{o[0] + v[0], o[1] + v[1], o[2] + v[2], o[3] + v[3]};
        }
        *dst = v;
        if constexpr (MODE == 2) {
          // the cotangent of the activation input from the stored activation and dY
          const floatx4 gy = ya[I];
          static_for<4>([&](auto c) {
            constexpr int C = decltype(c)::value;
            v[C] = act_grad(ACT, gy[C], v[C]);
          });
          *reinterpret_cast<floatx4*>(p.dz + row * p.ldaux + col_e) = v;
        }
        static_for<4>([&](auto c) { cs[decltype(c)::value] += (double)v[decltype(c)::value]; });
      });
    }
  };
  auto by_acc = [&](auto modec, auto actc) {
    if (p.accumulate) store_rows(modec, actc, std::true_type{});
    else store_rows(modec, actc, std::false_type{});
  };
  auto by_act = [&](auto modec) {
    switch (p.act) {
      case ACT_RELU: by_acc(modec, std::integral_constant<int, ACT_RELU>{}); break;
      case ACT_TANH: by_acc(modec, std::integral_constant<int, ACT_TANH>{}); break;
      case ACT_SIGMOID: by_acc(modec, std::integral_constant<int, ACT_SIGMOID>{}); break;
      default: by_acc(modec, std::integral_constant<int, ACT_NONE>{}); break;
    }
  };
  if (p.mode == 0) by_act(std::integral_constant<int, 0>{});
  else if (p.mode == 1) by_act(std::integral_constant<int, 1>{});
  else by_act(std::integral_constant<int, 2>{});
  if (p.colsum_partial != nullptr) {
    // lanes q + ECPR rg hold the same columns: one partial row per wave
    static_for<4>([&](auto c) {
      constexpr int C = decltype(c)::value;
      for (int o = ECPR; o < 64; o <<= 1) cs[C] += __shfl_xor(cs[C], o, 64);
    });
    if (rg == 0 && col_ok) {
      // one partial row per wave row and K group
      double* dst = p.colsum_partial + (((int64_t)tm * 2 + wm) * KS + kgroup) * p.N + col_e;
      static_for<4>([&](auto c) { dst[decltype(c)::value] = cs[decltype(c)::value]; });
    }
  }
}

// The direct-to-LDS kernel is on unless SHK_HIP_GEMM_V2=0 (read once per process).
inline bool v2_enabled() {
  static const bool on = [] {
    const char* e = getenv("SHK_HIP_GEMM_V2");
    return e == nullptr || atoi(e) != 0;
  }();
  return on;
}

// In-workgroup split-K is on unless SHK_HIP_GEMM_KS2=0 (read once per process).
inline bool v2_ks2_enabled() {
  static const bool on = [] {
    const char* e = getenv("SHK_HIP_GEMM_KS2");
    return e == nullptr || atoi(e) != 0;
  }();
  return on;
}

// Kernel choice for a GEMM (0: none, the register-staged kernel runs it; else the tile edge).
//   * both operands allow 16-byte loads, K and N are multiples of 4 and, for the transposed
//     epilogue, its pointers are 16-byte aligned with leading dimensions multiples of 4;
//   * BT = 128 when there are at least 256 such tiles (times split-K slices);
//   * BT = 64 for problems with at least 128 64x64 tiles and K <= 2048 that are not split, in
//     place of splitting K (no partials, no reduction pass).
// TAIL variants run when M, N or K (or the slice) is not a whole number of tiles.
inline int v2_choose(const GemmParams& p, bool va, bool vb) {
  if (!va || !vb || p.K % 4 != 0 || p.N % 4 != 0 || p.K < 4) return 0;
  auto al = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; };
  if (p.kchunk > 0) {
    if (p.kchunk % V2_BK != 0 || p.partial == nullptr) return 0;
  } else if (p.upd.pn != nullptr) {
    const GemmUpdate& u = p.upd;
    if (!al(u.p) || !al(u.pn) || (u.m != nullptr && (!al(u.m) || !al(u.mn))) ||
        (u.kind != 0 && (!al(u.v) || !al(u.vn))))
      return 0;
  } else {
    if (!al(p.C) || p.ldc % 4 != 0 || (p.bias != nullptr && !al(p.bias))) return 0;
    if (p.mode != 0 && (!al(p.aux) || p.ldaux % 4 != 0)) return 0;
    if (p.mode == 2 && !al(p.dz)) return 0;
  }
  const int64_t ld = std::max(p.lda, p.ldb);
  if ((p.M + 128) * ld >= (1LL << 31) || (p.N + 128) * ld >= (1LL << 31) ||
      (p.K + 128) * ld >= (1LL << 31))
    return 0;
  const int64_t slices = p.kchunk > 0 ? (p.K + p.kchunk - 1) / p.kchunk : 1;
  const int64_t t128 = ((p.M + 127) / 128) * ((p.N + 127) / 128);
  const int64_t t64 = ((p.M + 63) / 64) * ((p.N + 63) / 64);
  if (t64 >= (1LL << 31) || slices >= 65536) return 0;
  if (t128 * slices >= 256) return 128;
  if (p.kchunk == 0 && t64 >= 128 && p.K <= 2048) return 64;
  return 0;
}

// In-workgroup split-K (KS = 2) for 64x64 tiles: fewer than two tiles per CU and at least
// eight k-tiles per group.
inline bool v2_split_in_group(const GemmParams& p, int bt) {
  const int64_t t64 = ((p.M + 63) / 64) * ((p.N + 63) / 64);
  return v2_ks2_enabled() && bt == 64 && p.kchunk == 0 && t64 < 512 && p.K >= 16 * V2_BK;
}

// In-workgroup split-K (KS = 2) for the split-K slices of 128x128 tiles: at most one workgroup
// per CU (fewer than 512 tile slices) and at least eight k-tiles per group. Eight waves give each
// SIMD two, as two four-wave workgroups per CU would, without more slices in HBM.
inline bool v2_split_slices_in_group(const GemmParams& p, unsigned tiles, unsigned slices) {
  return v2_ks2_enabled() && p.kchunk > 0 && p.partial != nullptr &&
         (int64_t)tiles * slices < 512 && p.kchunk >= 16 * V2_BK;
}

template <bool TA, bool TB, int BT>
hipError_t launch_v2_bt(const GemmParams& p, hipStream_t s) {
  g_colsum_rows = ((p.M + BT - 1) / BT) * 2;
  const unsigned tiles = (unsigned)(((p.M + BT - 1) / BT) * ((p.N + BT - 1) / BT));
  const unsigned slices = p.kchunk > 0 ? (unsigned)((p.K + p.kchunk - 1) / p.kchunk) : 1u;
  const int64_t span = p.kchunk > 0 ? p.kchunk : p.K;
  if constexpr (BT == 64) {
    if (v2_split_in_group(p, BT)) {
      g_colsum_rows = ((p.M + BT - 1) / BT) * 4;  // per wave row and K group
      // both groups whole k-tiles only when K is a multiple of 2 BK
      const bool tail = p.M % BT != 0 || p.N % BT != 0 || p.K % (2 * V2_BK) != 0;
      if (tail)
        hipLaunchKernelGGL((gemm_f32_v2<!TA, TB, BT, true, 2>), dim3(tiles), dim3(2 * V2_NT), 0,
                           s, p);
      else
        hipLaunchKernelGGL((gemm_f32_v2<!TA, TB, BT, false, 2>), dim3(tiles), dim3(2 * V2_NT), 0,
                           s, p);
      return hipGetLastError();
    }
  }
  const bool tail = p.M % BT != 0 || p.N % BT != 0 || span % V2_BK != 0 || p.K % V2_BK != 0;
  if constexpr (BT == 128) {
    if (v2_split_slices_in_group(p, tiles, slices)) {
      // both groups whole k-tiles of every slice only when every slice, the last included, is a
      // multiple of 2 BK
      const bool tail2 = tail || span % (2 * V2_BK) != 0 ||
                         (p.K - (int64_t)(slices - 1) * span) % (2 * V2_BK) != 0;
      if (tail2)
        hipLaunchKernelGGL((gemm_f32_v2<!TA, TB, BT, true, 2>), dim3(tiles, slices),
                           dim3(2 * V2_NT), 0, s, p);
      else
        hipLaunchKernelGGL((gemm_f32_v2<!TA, TB, BT, false, 2>), dim3(tiles, slices),
                           dim3(2 * V2_NT), 0, s, p);
      return hipGetLastError();
    }
  }
  if (tail)
    hipLaunchKernelGGL((gemm_f32_v2<!TA, TB, BT, true, 1>), dim3(tiles, slices), dim3(V2_NT), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_f32_v2<!TA, TB, BT, false, 1>), dim3(tiles, slices), dim3(V2_NT), 0, s, p);
  return hipGetLastError();
}

template <bool TA, bool TB>
hipError_t launch_v2(const GemmParams& p, int bt, hipStream_t s) {
  return bt == 64 ? launch_v2_bt<TA, TB, 64>(p, s) : launch_v2_bt<TA, TB, 128>(p, s);
}

}  // namespace
}  // namespace shk
