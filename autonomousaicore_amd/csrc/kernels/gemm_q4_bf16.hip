// GEMM kernels with the INT4 B operand (QLoRA base weights dequantized in the kernel), bf16 output.
#include "gemm_kernels.inc"

AIC_GEMM_Q4_CT(aic::hip::bf16)
