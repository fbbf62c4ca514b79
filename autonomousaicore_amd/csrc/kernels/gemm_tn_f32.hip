// GEMM kernels for the operand layout op(A) = A^T, op(B) = B: the weight gradient (true, false), fp32 output.
#include "gemm_kernels.inc"

AIC_GEMM_LAUNCHES_CT(true, false, float)
AIC_GEMM_RAGGED_CT(true, false, float)
