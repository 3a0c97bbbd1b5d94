// fp32 MFMA GEMM tile kernels for the NT layout (transA = 0, transB = 1).
#define SHK_TA false
#define SHK_TB true
#include "gemm_layout.inc"
