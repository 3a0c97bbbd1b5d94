// fp32 MFMA GEMM tile kernels for the TN layout (transA = 1, transB = 0).
#define SHK_TA true
#define SHK_TB false
#include "gemm_layout.inc"
