// QLoRA projection: a frozen INT4-symmetric base weight plus a trainable LoRA adapter,
//   y = x . deq(Wq)^T + ((x . A^T) . B^T) * (alpha / rank)  [+ R],
// the composition of QuantizedLinear::forward (src/nn/quantization.cpp:669-679) as the base of
// LoRALinear::forward (src/nn/lora.cpp:75-93), which the QLoRA configuration applies to every
// q/k/v/out/gate/up/down projection.  The base weight receives no gradient (lora.cpp:54-56).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../runtime/dtype.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::models {

// C[M,N] = alpha * X . op(deq(Wq)) + beta * C + R.  transW = 1: Wq holds W [N, K] (forward,
// x W^T); transW = 0: Wq holds W [K, N] (input gradient, dy W).  Groups run along W's flat
// row-major index.  bf16 operands in the shapes the GEMM kernel takes (K % 64, group % 64, the
// weight's row length % 64, N % 64 for dy W): dequantized inside the GEMM's operand load.
// Otherwise (fp32 operands, other shapes) the weight is dequantized into a pool buffer of the
// operand type first.  Either way op(B) holds bf16(q * scale) (fp32 operands: q * scale).
void int4_dequant_gemm(int transW, int64_t M, int64_t N, int64_t K, float alpha, const void* X, int64_t ldx,
                       const uint8_t* Wq, const void* scales, DType scale_t, int64_t group, float beta, void* C,
                       int64_t ldc, const void* R, int64_t ldr, DType ab, DType c, hipStream_t s);

class QLoRALinear {
public:
    // rank may be 0 (the plain QuantizedLinear).  dt: operand and output type (f32 or bf16).
    QLoRALinear(int64_t in, int64_t out, int64_t rank, float alpha, int64_t group, DType scale_t, DType dt);

    float scaling() const { return rank_ > 0 ? alpha_ / static_cast<float>(rank_) : 0.0f; }

    // x [T, in], A [rank, in], B [out, rank], R / y [T, out], all dt and contiguous.  Wq, scales,
    // x, A and B stay referenced until backward.
    void forward(const void* x, int64_t T, const uint8_t* Wq, const void* scales, const void* A, const void* B,
                 const void* R, void* y, hipStream_t s);
    // dy [T, out] (dt) -> dx [T, in] (dt, overwritten; may be null), dA [rank, in] and dB [out, rank]
    // (fp32; overwritten, or added to when accumulate).
    void backward(const void* dy, void* dx, float* dA, float* dB, bool accumulate, hipStream_t s);

private:
    int64_t in_, out_, rank_, group_;
    float alpha_;
    DType scale_t_, dt_;
    int64_t T_ = 0;
    const void* x_ = nullptr;
    const void* A_ = nullptr;
    const void* B_ = nullptr;
    const uint8_t* Wq_ = nullptr;  // the frozen base, read again (dequantized) by backward
    const void* scales_ = nullptr;
    DeviceBuffer xa_;
};

}  // namespace aic::models
