// Skinny-GEMM routes (one of M, N, K at most 16) and the split-K finishing pass they share with
// the tile kernels. Implemented in gemm_skinny.hip and gemm.hip.
#pragma once
#include "kernels.h"

namespace shk {

enum SkinnyRoute { SKINNY_NONE = 0, SKINNY_SMALL_K, SKINNY_ROW_DOT, SKINNY_COL_OUTER };

// SHK_HIP_GEMM_SKINNY=0 routes every GEMM to the tile kernels (for comparisons).
bool skinny_enabled();
SkinnyRoute skinny_route(const GemmParams& p);
// Row blocks of the small-K kernel (also the number of column-sum partial rows it writes).
constexpr int64_t SMALL_K_MAX_ROW_BLOCKS = 128;
int64_t small_k_row_blocks(int64_t M, int64_t N);
// K panels of the column-outer kernel for `cols` wide columns.
int64_t skinny_outer_slices(int64_t cols, int64_t K);
// Partial floats the column-outer route may need for an M x N x K problem (either operand wide).
int64_t skinny_workspace_floats(int64_t M, int64_t N, int64_t K);
// Runs the GEMM on `route` (!= SKINNY_NONE); the column-outer route writes its panel sums to
// `workspace`, which must hold skinny_workspace_floats(M, N, K) floats.
hipError_t launch_skinny(const GemmParams& p, SkinnyRoute route, float* workspace, hipStream_t s);
// Sums `slices` partial planes p.partial[slice][M][N] in slice order and applies the epilogue.
hipError_t launch_splitk_finish(const GemmParams& p, int slices, hipStream_t s);

}  // namespace shk
