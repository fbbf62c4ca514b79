// GEMM kernels for the operand layout op(A) = A, op(B) = B^T: the Linear forward (false, true), bf16 output.
#include "gemm_kernels.inc"

AIC_GEMM_LAUNCHES_CT(false, true, aic::hip::bf16)
AIC_GEMM_RAGGED_CT(false, true, aic::hip::bf16)
