// fp32 MFMA GEMM tile kernels for the NN layout (transA = 0, transB = 0).
#define SHK_TA false
#define SHK_TB false
#include "gemm_layout.inc"
