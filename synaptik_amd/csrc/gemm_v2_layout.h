// LDS layouts of the large-problem GEMM tile kernel (gemm_v2.h): where each 16-byte chunk of an
// operand tile lives in a stage, and the inverse map used to place the direct-to-LDS copies.
// A stage holds one BT x 32 operand tile (BT = 128 or 64: BT * 32 floats, BT * 8 chunks). Plain
// C++ so that the host tests can check the maps (tests/gemm_layout_harness.cpp defines __host__ /
// __device__ away).
#pragma once

namespace shk {

// LDS float offset of chunk c (k = 4c..4c+3) of row r in a K-contiguous tile: rows 2L and 2L+1
// share one 256-byte line whose 16 chunk slots are permuted by XOR with L mod 16.
__host__ __device__ constexpr int v2_kmaj_off(int r, int c) {
  return ((r >> 1) * 16 + ((((r & 1) << 3) | c) ^ ((r >> 1) & 15))) * 4;
}
// LDS float offset of element (k, m) in an M/N-contiguous tile: cpr = BT / 4 chunks of four per
// k-row (at least 16), chunk slot XORed with 4 * ((k / 4) mod 4), so the four lane groups of a
// fragment read (rows k = 16h + 4g + s) land on four different 16-bank groups.
__host__ __device__ constexpr int v2_mnmaj_off(int k, int m, int cpr) {
  return k * 4 * cpr + (((m >> 2) ^ (((k >> 2) & 3) << 2)) << 2) + (m & 3);
}

// Source of LDS chunk q (16 bytes; q in [0, BT * 8)) of a stage, inverse of the layouts above:
// K-contiguous tiles hold chunk c (k = 4c..4c+3) of row r; M/N-contiguous tiles hold chunk c
// (rows 4c..4c+3) of k-row k. Returned as r * 8 + c (K-contiguous) or k * cpr + c
// (M/N-contiguous).
__host__ __device__ constexpr int v2_kmaj_src(int q) {
  return (2 * (q >> 4) + ((((q & 15) ^ ((q >> 4) & 15)) >> 3))) * 8 + (((q & 15) ^ ((q >> 4) & 15)) & 7);
}
__host__ __device__ constexpr int v2_mnmaj_src(int q, int cpr) {
  return (q / cpr) * cpr + ((q % cpr) ^ ((((q / cpr) >> 2) & 3) << 2));
}

}  // namespace shk
