// GEMM kernels for the operand layout op(A) = A^T, op(B) = B^T (true, true), fp32 output.
#include "gemm_kernels.inc"

AIC_GEMM_LAUNCHES_CT(true, true, float)
