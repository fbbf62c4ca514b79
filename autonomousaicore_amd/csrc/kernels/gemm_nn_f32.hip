// GEMM kernels for the operand layout op(A) = A, op(B) = B: the input gradient (false, false), fp32 output.
#include "gemm_kernels.inc"

AIC_GEMM_LAUNCHES_CT(false, false, float)
AIC_GEMM_RAGGED_CT(false, false, float)
