// Large-problem fp32 MFMA GEMM tile kernel for gfx950: 128x128 output tiles, BK = 32, four
// waves of 64x64, v_mfma_f32_16x16x4_f32, operands moved from HBM straight into LDS.
//
// Used when M and N are multiples of 128, K a multiple of 32, both operands allow 16-byte
// loads and the problem has at least 256 output tiles (the MLP-4096 and C2-sized GEMMs); every
// other case runs the register-staged kernel in gemm_tile.h. The epilogues are the same: bias +
// activation, activation gradient, accumulate, the binary64 column-sum partials of a bias
// gradient, and the staged optimizer update of a weight gradient.
//
// Data movement:
//   * global_load_lds_dwordx4: each lane copies 16 bytes from HBM to LDS without passing through
//     VGPRs; one wave instruction fills 1 KB of LDS. The lane -> address assignment inside an
//     instruction is free, which is used to lay the tile out swizzled (below). Two LDS stages,
//     software-pipelined so that fragment reads overlap MFMAs and each copy has a whole k-tile
//     of MFMA work to land; one barrier per 32-deep k-tile (see the main loop).
//   * K-contiguous operands (A = X[M,K], B = W[N,K]) are kept [row][k] with 16-byte chunks
//     XOR-swizzled across each 256-byte pair of rows, so that one ds_read_b128 per lane fetches
//     four k values of a row and the 64 lanes of a read hit 64 distinct banks.
//   * M/N-contiguous operands (dZ^T, X, W in [K,N]) are kept [k][row] with chunks swizzled by
//     (k / 4) mod 4; fragments are ds_read_b32.
// Reduction order: within a 32-deep k-tile, MFMA s of half h takes k = 16h + 4g + s from lane
// group g; the sum over k is a permutation of the straight order, which the matrix cores
// reassociate anyway (the reference contract allows it, foundational-modules.md:423-425).
#pragma once
#include "gemm_tile.h"
#include "gemm_v2_layout.h"

namespace shk {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int V2_BM = 128, V2_BN = 128, V2_BK = 32, V2_NT = 256;
constexpr int V2_TILE = 128 * 32;  // floats per operand per stage

// Per-lane source offsets (bytes, relative to the tile origin) of the four 16-byte copies this
// thread issues per operand per k-tile, and where they land.
template <bool KMAJ>
struct V2Loader {
  uint32_t voff[4];
  uint32_t wdst;  // this wave's byte offset inside a stage (wave-uniform)
  __device__ __forceinline__ void init(int64_t ld) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    wdst = __builtin_amdgcn_readfirstlane((uint32_t)w * 1024u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = (i * 4 + w) * 64 + lane;  // destination chunk of this lane
      if constexpr (KMAJ) {
        const int src = v2_kmaj_src(q), r = src >> 3, c = src & 7;
        voff[i] = (uint32_t)((r * ld + 4 * c) * 4);
      } else {
        const int src = v2_mnmaj_src(q), k = src >> 5, c = src & 31;
        voff[i] = (uint32_t)((k * ld + 4 * c) * 4);
      }
    }
  }
  // Copy I of this wave for the k-tile whose element (row 0, k 0) is `tile`, into stage `lds`:
  // global_load_lds_dwordx4 with the tile origin in SGPRs, a per-lane 32-bit offset and the LDS
  // destination in M0.
  // Written as inline assembly so that the compiler does not track the copies (it would make
  // every LDS read wait for all copies in flight, including those into the other stage); the
  // kernel waits for them itself (v2_wait_all) before each barrier.
  template <int I>
  __device__ __forceinline__ void issue(const float* tile, float* lds) const {
    const uint32_t dst =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)lds + I * 4096u + wdst;
    asm volatile("global_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff[I]), "s"(tile), "{m0}"(dst)
                 : "memory");
  }
};

// Fragments of one operand for one half (16 k) of a k-tile: f[b][s] is the value lane
// (row 16b + lane % 16 of the wave's sub-tile; group g = lane / 16) supplies to MFMA s.
template <bool KMAJ>
struct V2Frag {
  floatx4 f[4];
  // K-contiguous: base[0] / base[1] are the offsets of this lane's chunk (4H + g) in the wave's
  // rows 0..15 / 16..31; blocks 2 and 3 repeat them 32 rows (1024 floats) further.
  // M/N-contiguous: base[b] = 512 g + 64 w + 16 (b ^ g) + l16; the k-row is compile-time.
  template <int H, int B>
  __device__ __forceinline__ void load_block(const float* lds, const int* base) {
    if constexpr (KMAJ) {
      f[B] = *reinterpret_cast<const floatx4*>(lds + base[B & 1] + (B >> 1) * 1024);
    } else {
      static_for<4>([&](auto s) {
        constexpr int S = decltype(s)::value;
        f[B][S] = lds[base[B] + (16 * H + S) * 128];
      });
    }
  }
  template <int H>
  __device__ __forceinline__ void load(const float* lds, const int* base) {
    static_for<4>([&](auto b) { load_block<H, decltype(b)::value>(lds, base); });
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
// along k (B stored [N,K]).
template <bool KA, bool KB>
__global__ void __launch_bounds__(V2_NT) __attribute__((amdgpu_waves_per_eu(2)))
gemm_f32_v2(GemmParams p) {
  __shared__ __attribute__((aligned(16))) float As0[V2_TILE];
  __shared__ __attribute__((aligned(16))) float Bs0[V2_TILE];
  __shared__ __attribute__((aligned(16))) float As1[V2_TILE];
  __shared__ __attribute__((aligned(16))) float Bs1[V2_TILE];

  const int tilesM = (int)(p.M / V2_BM), tilesN = (int)(p.N / V2_BN);
  int tm, tn;
  tile_of(blockIdx.x, tilesM, tilesN, tm, tn);
  const int64_t m0 = (int64_t)tm * V2_BM, n0 = (int64_t)tn * V2_BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, g = lane >> 4;

  // operand tile origins at k = 0, and the per-k-tile advance
  // split-K: block row y covers k in [y * kchunk, min(K, (y + 1) * kchunk))
  const int64_t k_begin = p.kchunk > 0 ? (int64_t)blockIdx.y * p.kchunk : 0;
  const int64_t k_len = p.kchunk > 0 ? std::min<int64_t>(p.kchunk, p.K - k_begin) : p.K;
  const float* a_tile = KA ? p.A + m0 * p.lda + k_begin : p.A + m0 + k_begin * p.lda;
  const float* b_tile = KB ? p.B + n0 * p.ldb + k_begin : p.B + n0 + k_begin * p.ldb;
  const int64_t a_step = KA ? V2_BK : V2_BK * p.lda;
  const int64_t b_step = KB ? V2_BK : V2_BK * p.ldb;
  V2Loader<KA> la;
  V2Loader<KB> lb;
  la.init(p.lda);
  lb.init(p.ldb);

  // lane-dependent fragment offsets per half
  int a_base[2][4], b_base[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a_base[h][q] = KA ? v2_kmaj_off(wm * 64 + 16 * (q & 1) + l16, 4 * h + g)
                        : 512 * g + 64 * wm + 16 * (q ^ g) + l16;
      b_base[h][q] = KB ? v2_kmaj_off(wn * 64 + 16 * (q & 1) + l16, 4 * h + g)
                        : 512 * g + 64 * wn + 16 * (q ^ g) + l16;
    }
  }

  floatx4 acc[4][4];
  static_for<4>([&](auto i) {
    static_for<4>([&](auto j) {
      acc[decltype(i)::value][decltype(j)::value] = floatx4{0.f, 0.f, 0.f, 0.f};
    });
  });

  const int nk = (int)(k_len / V2_BK);
  // 64 MFMAs of one half-tile in 8 groups of 8 (group q: MFMA s = q / 2 of blocks
  // i = 2 (q % 2) .. +1, j = 0..3); after each group, side(q) issues that group's share of the
  // LDS reads and copies. The scheduling barriers keep this order: reads and copies spread over
  // the MFMA stream instead of stalling it in one place.
  auto mfma_half = [&](const V2Frag<KA>& fa, const V2Frag<KB>& fb, auto side) {
    static_for<8>([&](auto q) {
      constexpr int Q = decltype(q)::value, S = Q >> 1, I0 = 2 * (Q & 1);
      static_for<2>([&](auto ii) {
        static_for<4>([&](auto j) {
          constexpr int I = I0 + decltype(ii)::value, J = decltype(j)::value;
          acc[I][J] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.f[I][S], fb.f[J][S], acc[I][J], 0,
                                                          0, 0);
        });
      });
      __builtin_amdgcn_sched_barrier(0);
      side(q);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // Fragment reads of half H from stage (As, Bs), two blocks per call for q = 0..3, ordered so
  // that the blocks the next half's first MFMAs use come first.
  auto read_share = [&](auto q, V2Frag<KA>& fa, V2Frag<KB>& fb, const float* As,
                        const float* Bs, auto h) {
    constexpr int Q = decltype(q)::value, H = decltype(h)::value;
    const int* ab = a_base[H];
    const int* bb = b_base[H];
    if constexpr (Q == 0) { fa.template load_block<H, 0>(As, ab); fb.template load_block<H, 0>(Bs, bb); }
    if constexpr (Q == 1) { fb.template load_block<H, 1>(Bs, bb); fa.template load_block<H, 1>(As, ab); }
    if constexpr (Q == 2) { fb.template load_block<H, 2>(Bs, bb); fb.template load_block<H, 3>(Bs, bb); }
    if constexpr (Q == 3) { fa.template load_block<H, 2>(As, ab); fa.template load_block<H, 3>(As, ab); }
  };

  // Software pipeline over k-tiles (tile kt lives in stage kt % 2; fa0 / fb0 hold its first-half
  // fragments on entry):
  //   first half: MFMAs with fa0 / fb0 while the second-half fragments load into fa1 / fb1;
  //   wait for this wave's copies and reads, barrier: tile kt+1 has landed everywhere and every
  //   wave has read all of tile kt;
  //   second half: MFMAs with fa1 / fb1 while tile kt+1's first-half fragments load into
  //   fa0 / fb0 (groups 0-3) and tile kt+2 is copied into tile kt's stage (groups 4-7).
  // Each copy has most of a k-tile of MFMA work to land; no LDS read touches a stage while a
  // copy into it is in flight.
  V2Frag<KA> fa0, fa1;
  V2Frag<KB> fb0, fb1;
  auto issue_all = [&](const float* at, const float* bt, float* As, float* Bs) {
    la.template issue<0>(at, As); la.template issue<1>(at, As);
    la.template issue<2>(at, As); la.template issue<3>(at, As);
    lb.template issue<0>(bt, Bs); lb.template issue<1>(bt, Bs);
    lb.template issue<2>(bt, Bs); lb.template issue<3>(bt, Bs);
  };
  issue_all(a_tile, b_tile, As0, Bs0);
  if (nk > 1) {
    issue_all(a_tile + a_step, b_tile + b_step, As1, Bs1);
    __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8): the first tile's eight copies have landed
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
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(fa0, fb0, [&](auto q) {
      if constexpr (decltype(q)::value < 4)
        read_share(q, fa1, fb1, Acur, Bcur, std::integral_constant<int, 1>{});
    });
    if (more) {
      v2_wait_all();
      v2_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(fa1, fb1, [&](auto q) {
      constexpr int Q = decltype(q)::value;
      if constexpr (Q < 4) {
        if (more) read_share(q, fa0, fb0, Aoth, Both, std::integral_constant<int, 0>{});
      } else {
        if (copy) {
          la.template issue<Q - 4>(at, Acur);
          lb.template issue<Q - 4>(bt, Bcur);
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
  // wave's 64x64 sub-tile. Split-K partials are written from that layout directly; otherwise
  // the sub-tile is transposed through this wave's own 16 KB of LDS (row-major, 16-byte chunks
  // XOR-swizzled by row) so that every global access of the epilogue is a 16-byte row segment:
  // lane (q = lane % 16, rg = lane / 16) then owns columns 4q..4q+3 of rows rg + 4t, t < 16,
  // and each store instruction writes four full 256-byte row segments.
  const int64_t row_w = m0 + wm * 64 + 4 * g, col_w = n0 + wn * 64 + l16;
  if (p.partial != nullptr) {
    // split-K: raw partial sums, reduced (and given the epilogue) by gemm_splitk_reduce
    float* part = p.partial + (int64_t)blockIdx.y * p.M * p.N;
    static_for<4>([&](auto i) {
      static_for<4>([&](auto j) {
        constexpr int I = decltype(i)::value, J = decltype(j)::value;
        float* dst = part + (row_w + 16 * I) * p.N + col_w + 16 * J;
        static_for<4>([&](auto r) { dst[decltype(r)::value * p.N] = acc[I][J][decltype(r)::value]; });
      });
    });
    return;
  }
  v2_wait_all();
  v2_barrier();  // every wave has finished reading its fragments: the stages are free
  float* stage = wave == 0 ? As0 : wave == 1 ? Bs0 : wave == 2 ? As1 : Bs1;
  static_for<4>([&](auto i) {
    static_for<4>([&](auto j) {
      constexpr int I = decltype(i)::value, J = decltype(j)::value;
      static_for<4>([&](auto r) {
        constexpr int R = decltype(r)::value;
        const int row = 16 * I + 4 * g + R, col = 16 * J + l16;
        stage[row * 64 + (((col >> 2) ^ (row & 15)) << 2) + (col & 3)] = acc[I][J][R];
      });
    });
  });
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are complete
  const int q = lane & 15, rg = lane >> 4;
  auto tile_row = [&](int t) -> floatx4 {
    const int row = rg + 4 * t;
    return *reinterpret_cast<const floatx4*>(stage + row * 64 + ((q ^ (row & 15)) << 2));
  };
  const int64_t row_e = m0 + wm * 64 + rg, col_e = n0 + wn * 64 + 4 * q;
  if (p.upd.pn != nullptr) {
    const GemmUpdate& u = p.upd;
    const UpdateCtx uc = update_ctx(u);
    bool ok = uc.k.ok;
    for (int t = 0; t < 16; ++t) {
      const int64_t e = (row_e + 4 * t) * p.N + col_e;
      const floatx4 gv = tile_row(t);
      const floatx4 pv = *reinterpret_cast<const floatx4*>(u.p + e);
      const floatx4 mv = u.m != nullptr ? *reinterpret_cast<const floatx4*>(u.m + e) : floatx4{0.f, 0.f, 0.f, 0.f};
      const floatx4 vv = u.kind != 0 ? *reinterpret_cast<const floatx4*>(u.v + e) : floatx4{0.f, 0.f, 0.f, 0.f};
      floatx4 pc, mc, vc = floatx4{0.f, 0.f, 0.f, 0.f};
      static_for<4>([&](auto c) {
        constexpr int C = decltype(c)::value;
        float pe, me, ve = 0.0f;
        if (u.kind == 0) ok &= sgd_element(u, uc.first, pv[C], gv[C], mv[C], pe, me);
        else ok &= adam_element(u, uc.k, pv[C], gv[C], mv[C], vv[C], pe, me, ve);
        pc[C] = pe;
        mc[C] = me;
        vc[C] = ve;
      });
      *reinterpret_cast<floatx4*>(u.pn + e) = pc;
      if (u.mn != nullptr) *reinterpret_cast<floatx4*>(u.mn + e) = mc;
      if (u.kind != 0) *reinterpret_cast<floatx4*>(u.vn + e) = vc;
    }
    update_flag(u, uc, ok);
    return;
  }
  floatx4 bias = floatx4{0.f, 0.f, 0.f, 0.f};
  if (p.bias != nullptr) bias = *reinterpret_cast<const floatx4*>(p.bias + col_e);
  double cs[4] = {0.0, 0.0, 0.0, 0.0};  // fused column sums of this lane's stored values
  for (int t = 0; t < 16; ++t) {
    const int64_t row = row_e + 4 * t;
    floatx4 v = tile_row(t);
    if (p.mode == 0) {
      if (p.bias != nullptr) v = floatx4{v[0] + bias[0], v[1] + bias[1], v[2] + bias[2], v[3] + bias[3]};
      static_for<4>([&](auto c) { v[decltype(c)::value] = apply_act(p.act, v[decltype(c)::value]); });
    } else {
      const floatx4 y = *reinterpret_cast<const floatx4*>(p.aux + row * p.ldaux + col_e);
      static_for<4>([&](auto c) {
        constexpr int C = decltype(c)::value;
        v[C] = act_grad(p.act, v[C], y[C]);
      });
    }
    floatx4* dst = reinterpret_cast<floatx4*>(p.C + row * p.ldc + col_e);
    if (p.accumulate) {
      const floatx4 o = *dst;
      v = floatx4{o[0] + v[0], o[1] + v[1], o[2] + v[2], o[3] + v[3]};
    }
    *dst = v;
    static_for<4>([&](auto c) { cs[decltype(c)::value] += (double)v[decltype(c)::value]; });
  }
  if (p.colsum_partial != nullptr) {
    // lanes q + 16 rg hold the same columns: one partial row per wave
    static_for<4>([&](auto c) {
      constexpr int C = decltype(c)::value;
      cs[C] += __shfl_xor(cs[C], 16, 64);
      cs[C] += __shfl_xor(cs[C], 32, 64);
    });
    if (rg == 0) {
      double* dst = p.colsum_partial + ((int64_t)tm * 2 + wm) * p.N + col_e;
      static_for<4>([&](auto c) { dst[decltype(c)::value] = cs[decltype(c)::value]; });
    }
  }
}

// Whether the large-problem kernel handles this GEMM (see the header comment): whole tiles,
// whole 32-deep k-tiles (per split-K slice when p.kchunk > 0), 16-byte operand loads, and
// enough workgroups to fill the chip (output tiles times slices).
inline bool v2_eligible(const GemmParams& p, bool va, bool vb) {
  if (!va || !vb || p.M % V2_BM != 0 || p.N % V2_BN != 0 || p.K % V2_BK != 0 || p.K < V2_BK)
    return false;
  if (p.kchunk > 0 && (p.kchunk % V2_BK != 0 || p.partial == nullptr)) return false;
  // the transposed epilogue moves 16-byte row segments
  auto al = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; };
  if (p.kchunk == 0) {
    if (p.upd.pn != nullptr) {
      const GemmUpdate& u = p.upd;
      if (!al(u.p) || !al(u.pn) || (u.m != nullptr && (!al(u.m) || !al(u.mn))) ||
          (u.kind != 0 && (!al(u.v) || !al(u.vn))))
        return false;
    } else {
      if (!al(p.C) || p.ldc % 4 != 0 || (p.bias != nullptr && !al(p.bias))) return false;
      if (p.mode == 1 && (!al(p.aux) || p.ldaux % 4 != 0)) return false;
    }
  }
  const int64_t tiles = (p.M / V2_BM) * (p.N / V2_BN);
  const int64_t slices = p.kchunk > 0 ? (p.K + p.kchunk - 1) / p.kchunk : 1;
  return tiles * slices >= 256 && tiles < (1LL << 31) && slices < 65536 &&
         p.M * std::max(p.lda, p.ldb) < (1LL << 31) && p.K * std::max(p.lda, p.ldb) < (1LL << 31);
}

template <bool TA, bool TB>
hipError_t launch_v2(const GemmParams& p, hipStream_t s) {
  g_colsum_rows = (p.M / V2_BM) * 2;
  const unsigned tiles = (unsigned)((p.M / V2_BM) * (p.N / V2_BN));
  const unsigned slices = p.kchunk > 0 ? (unsigned)((p.K + p.kchunk - 1) / p.kchunk) : 1u;
  hipLaunchKernelGGL((gemm_f32_v2<!TA, TB>), dim3(tiles, slices), dim3(V2_NT), 0, s, p);
  return hipGetLastError();
}

}  // namespace
}  // namespace shk
