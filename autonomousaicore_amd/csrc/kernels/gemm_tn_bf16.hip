// GEMM kernels for the operand layout op(A) = A^T, op(B) = B: the weight gradient (true, false), bf16 output.
#include "gemm_kernels.inc"

AIC_GEMM_LAUNCHES_CT(true, false, aic::hip::bf16)
AIC_GEMM_RAGGED_CT(true, false, aic::hip::bf16)
