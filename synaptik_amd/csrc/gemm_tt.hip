// fp32 MFMA GEMM tile kernels for the TT layout (transA = 1, transB = 1).
#define SHK_TA true
#define SHK_TB true
#include "gemm_layout.inc"
