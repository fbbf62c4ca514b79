#include "qlora_linear.hpp"

#include "../kernels/gemm.hpp"
#include "../kernels/kernels.hpp"
#include "../runtime/error.hpp"

namespace aic::models {

namespace {

void gemm(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const void* A, int64_t lda, const void* B,
          int64_t ldb, float beta, void* C, int64_t ldc, DType ab, DType c, hipStream_t s, const void* R = nullptr,
          int64_t ldr = 0) {
    hip::GemmArgs a;
    a.transA = ta;
    a.transB = tb;
    a.M = M;
    a.N = N;
    a.K = K;
    a.alpha = alpha;
    a.A = A;
    a.lda = lda;
    a.B = B;
    a.ldb = ldb;
    a.beta = beta;
    a.C = C;
    a.ldc = ldc;
    a.R = R;
    a.ldr = ldr;
    a.ab = ab;
    a.c = c;
    hip::gemm(a, s);
}

// The product C = alpha X op(deq(Wq)) + beta C + R with the INT4 weight dequantized inside the
// GEMM kernel (GemmArgs::Bq), when the kernel takes the shape.
bool fused_q4(int transW, int64_t M, int64_t N, int64_t K, float alpha, const void* X, int64_t ldx, const uint8_t* Wq,
              const void* scales, DType scale_t, int64_t group, float beta, void* C, int64_t ldc, const void* R,
              int64_t ldr, DType ab, DType c, hipStream_t s) {
    hip::GemmArgs a;
    a.transA = 0;
    a.transB = transW ? 1 : 0;
    a.M = M;
    a.N = N;
    a.K = K;
    a.alpha = alpha;
    a.A = X;
    a.lda = ldx;
    a.ldb = transW ? K : N;
    a.beta = beta;
    a.C = C;
    a.ldc = ldc;
    a.R = R;
    a.ldr = ldr;
    a.ab = ab;
    a.c = c;
    a.Bq = Wq;
    a.Bscale = scales;
    a.scale_t = scale_t;
    a.group = hip::int4_group(N * K, group);
    if (!hip::gemm_q4_eligible(a)) return false;
    hip::gemm(a, s);
    return true;
}

void check_dt(DType ab, DType c, DType scale_t) {
    AIC_CHECK(ab == DType::Float32 || ab == DType::BFloat16, DTypeMismatch, "int4 GEMM: operands must be f32 or bf16");
    AIC_CHECK(c == DType::Float32 || c == DType::BFloat16, DTypeMismatch, "int4 GEMM: output must be f32 or bf16");
    AIC_CHECK(scale_t == DType::Float32 || scale_t == DType::Float16, DTypeMismatch, "int4: scales must be f32 or f16");
}

}  // namespace

void int4_dequant_gemm(int transW, int64_t M, int64_t N, int64_t K, float alpha, const void* X, int64_t ldx,
                       const uint8_t* Wq, const void* scales, DType scale_t, int64_t group, float beta, void* C,
                       int64_t ldc, const void* R, int64_t ldr, DType ab, DType c, hipStream_t s) {
    check_dt(ab, c, scale_t);
    AIC_CHECK(M >= 0 && N >= 0 && K >= 0, InvalidArgument, "int4_dequant_gemm: negative size");
    if (M == 0 || N == 0) return;
    AIC_CHECK(X && Wq && scales && C, InvalidArgument, "int4_dequant_gemm: null pointer");
    if (fused_q4(transW, M, N, K, alpha, X, ldx, Wq, scales, scale_t, group, beta, C, ldc, R, ldr, ab, c, s)) return;
    // other shapes and fp32 operands: the weight dequantized into a pool buffer first
    DeviceBuffer w(dtype_size(ab) * static_cast<size_t>(N * K > 0 ? N * K : 1), s);
    hip::int4_dequant(Wq, scales, scale_t, N * K, group, w.get(), ab, s);
    gemm(0, transW ? 1 : 0, M, N, K, alpha, X, ldx, w.get(), transW ? K : N, beta, C, ldc, ab, c, s, R, ldr);
}

QLoRALinear::QLoRALinear(int64_t in, int64_t out, int64_t rank, float alpha, int64_t group, DType scale_t, DType dt)
    : in_(in), out_(out), rank_(rank), group_(group), alpha_(alpha), scale_t_(scale_t), dt_(dt) {
    AIC_CHECK(in > 0 && out > 0 && rank >= 0, InvalidArgument, "QLoRALinear: need in, out > 0 and rank >= 0");
    check_dt(dt, dt, scale_t);
    hip::int4_group(in * out, group);  // rejects an odd multi-group size now
}

void QLoRALinear::forward(const void* x, int64_t T, const uint8_t* Wq, const void* scales, const void* A,
                          const void* B, const void* R, void* y, hipStream_t s) {
    AIC_CHECK(x && Wq && scales && y && T > 0, InvalidArgument, "QLoRALinear::forward: bad arguments");
    AIC_CHECK(rank_ == 0 || (A && B), InvalidArgument, "QLoRALinear::forward: null adapter");
    const size_t es = dtype_size(dt_);
    T_ = T;
    x_ = x;
    A_ = A;
    B_ = B;
    Wq_ = Wq;
    scales_ = scales;
    float beta = 0.0f;
    if (rank_ > 0) {
        xa_ = DeviceBuffer(es * static_cast<size_t>(T * rank_), s);
        gemm(0, 1, T, rank_, in_, 1.0f, x, in_, A, in_, 0.0f, xa_.get(), rank_, dt_, dt_, s);       // x A^T
        gemm(0, 1, T, out_, rank_, scaling(), xa_.get(), rank_, B, rank_, 0.0f, y, out_, dt_, dt_, s);  // * B^T * s
        beta = 1.0f;
    }
    int4_dequant_gemm(1, T, out_, in_, 1.0f, x, in_, Wq, scales, scale_t_, group_, beta, y, out_, R, out_, dt_, dt_,
                      s);  // + x deq(Wq)^T (+ R)
}

void QLoRALinear::backward(const void* dy, void* dx, float* dA, float* dB, bool accumulate, hipStream_t s) {
    AIC_CHECK(dy && T_ > 0 && Wq_, InvalidArgument, "QLoRALinear::backward: no forward to differentiate");
    AIC_CHECK(rank_ == 0 || (dA && dB), InvalidArgument, "QLoRALinear::backward: null adapter gradient");
    const float acc = accumulate ? 1.0f : 0.0f;
    float beta = 0.0f;
    if (rank_ > 0) {
        const float sc = scaling();
        DeviceBuffer dxa(dtype_size(dt_) * static_cast<size_t>(T_ * rank_), s);
        gemm(0, 0, T_, rank_, out_, sc, dy, out_, B_, rank_, 0.0f, dxa.get(), rank_, dt_, dt_, s);       // s dy B
        gemm(1, 0, out_, rank_, T_, sc, dy, out_, xa_.get(), rank_, acc, dB, rank_, dt_, DType::Float32, s);  // s dy^T xa
        gemm(1, 0, rank_, in_, T_, 1.0f, dxa.get(), rank_, x_, in_, acc, dA, in_, dt_, DType::Float32, s);     // dxa^T x
        if (dx) gemm(0, 0, T_, in_, rank_, 1.0f, dxa.get(), rank_, A_, in_, 0.0f, dx, in_, dt_, dt_, s);     // dxa A
        beta = 1.0f;
    }
    if (dx)
        int4_dequant_gemm(0, T_, in_, out_, 1.0f, dy, out_, Wq_, scales_, scale_t_, group_, beta, dx, in_, nullptr, 0,
                          dt_, dt_, s);  // + dy deq(Wq)
}

}  // namespace aic::models
