// GEMM kernels for the operand layout op(A) = A, op(B) = B: the input gradient (false, false), bf16 output.
#include "gemm_kernels.inc"

AIC_GEMM_LAUNCHES_CT(false, false, aic::hip::bf16)
AIC_GEMM_RAGGED_CT(false, false, aic::hip::bf16)
