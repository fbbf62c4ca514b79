// GEMM kernels for the operand layout op(A) = A, op(B) = B^T: the Linear forward (false, true), fp32 output.
#include "gemm_kernels.inc"

AIC_GEMM_LAUNCHES_CT(false, true, float)
AIC_GEMM_RAGGED_CT(false, true, float)
