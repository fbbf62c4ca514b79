// extern "C" boundary of the library (declared in include/aic_hip.h).  Every entry catches
// aic::Error / std::exception, records the message for aic_hip_last_error() and returns
// the error code; nothing throws across the ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <exception>
#include <new>
#include <string>

#include "../../../include/aic_hip.h"
#include "../data/synthetic.hpp"
#include "../data/token_data.hpp"
#include "../kernels/gemm.hpp"
#include "../kernels/kernels.hpp"
#include "../model/moe_ffn.hpp"
#include "../model/qlora_linear.hpp"
#include "../model/transformer_lm.hpp"
#include "../runtime/error.hpp"
#include "../runtime/memory_pool.hpp"
#include "../runtime/telemetry.hpp"

namespace aic {

const char* error_code_name(ErrorCode c) noexcept {
    switch (c) {
        case ErrorCode::Ok: return "Ok";
        case ErrorCode::InvalidArgument: return "InvalidArgument";
        case ErrorCode::OutOfRange: return "OutOfRange";
        case ErrorCode::ShapeMismatch: return "ShapeMismatch";
        case ErrorCode::DTypeMismatch: return "DTypeMismatch";
        case ErrorCode::DeviceMismatch: return "DeviceMismatch";
        case ErrorCode::OutOfMemory: return "OutOfMemory";
        case ErrorCode::HipError: return "HipError";
        case ErrorCode::NotImplemented: return "NotImplemented";
        case ErrorCode::BackendUnavailable: return "BackendUnavailable";
        case ErrorCode::IOError: return "IOError";
        case ErrorCode::FormatError: return "FormatError";
        case ErrorCode::Overflow: return "Overflow";
        case ErrorCode::InvalidState: return "InvalidState";
        case ErrorCode::RuntimeError: return "RuntimeError";
        case ErrorCode::Internal: return "Internal";
    }
    return "Unknown";
}

const char* dtype_name(DType d) noexcept {
    switch (d) {
        case DType::Float32: return "float32";
        case DType::Float16: return "float16";
        case DType::BFloat16: return "bfloat16";
        case DType::Int32: return "int32";
        case DType::Int64: return "int64";
        case DType::UInt8: return "uint8";
        case DType::UInt16: return "uint16";
    }
    return "unknown";
}

}  // namespace aic

struct aic_moe_ffn {
    aic::models::MoEFFN* ffn;
};

struct aic_qlora_linear {
    aic::models::QLoRALinear* lin;
};

struct aic_lm {
    aic::models::TransformerLM* model;
};

namespace {

thread_local std::string t_last_error;

template <typename F>
int guard(F&& f) {
    try {
        f();
        t_last_error.clear();
        return 0;
    } catch (const aic::Error& e) {
        t_last_error = e.what();
        return static_cast<int>(e.code());
    } catch (const std::bad_alloc& e) {
        t_last_error = std::string("host allocation failed: ") + e.what();
        return static_cast<int>(aic::ErrorCode::OutOfMemory);
    } catch (const std::exception& e) {
        t_last_error = e.what();
        return static_cast<int>(aic::ErrorCode::RuntimeError);
    } catch (...) {
        t_last_error = "unknown error";
        return static_cast<int>(aic::ErrorCode::Internal);
    }
}

aic::DType dt(aic_dtype d) { return static_cast<aic::DType>(static_cast<int>(d)); }
hipStream_t st(aic_stream s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

const char* aic_hip_last_error(void) { return t_last_error.c_str(); }

int aic_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

const char* aic_hip_version(void) { return "autonomousaicore_amd 0.1.0 (gfx950)"; }

int aic_hip_mem_alloc_async(void** ptr, size_t bytes, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(ptr, InvalidArgument, "null output pointer");
        *ptr = aic::pool_alloc(bytes, st(stream));
    });
}

int aic_hip_mem_free_async(void* ptr, aic_stream stream) { return guard([&] { aic::pool_free(ptr, st(stream)); }); }

int aic_hip_mem_release_stream(aic_stream stream) { return guard([&] { aic::stream_scratch_release(st(stream)); }); }

int aic_hip_mem_stats(int64_t* allocated_bytes, int64_t* peak_bytes) {
    return guard([&] {
        const aic::MemoryStats s = aic::pool_stats();
        if (allocated_bytes) *allocated_bytes = s.allocated_bytes;
        if (peak_bytes) *peak_bytes = s.peak_bytes;
    });
}

int aic_hip_gemm(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha, const void* A, int64_t lda,
                 const void* B, int64_t ldb, float beta, void* C, int64_t ldc, const void* R, int64_t ldr,
                 aic_dtype ab_type, aic_dtype c_type, aic_stream stream) {
    return guard([&] {
        aic::hip::GemmArgs a;
        a.transA = transA;
        a.transB = transB;
        a.M = M;
        a.N = N;
        a.K = K;
        a.alpha = alpha;
        a.beta = beta;
        a.A = A;
        a.lda = lda;
        a.B = B;
        a.ldb = ldb;
        a.C = C;
        a.ldc = ldc;
        a.R = R;
        a.ldr = ldr;
        a.ab = dt(ab_type);
        a.c = dt(c_type);
        aic::hip::gemm(a, st(stream));
    });
}

int aic_hip_gemm_lowrank(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha, const void* A,
                         int64_t lda, const void* B, int64_t ldb, const void* X2, int64_t ldx2, const void* Y2,
                         int64_t ldy2, int64_t r2, int64_t seg_n, int y2_kmajor, float beta, void* C, int64_t ldc,
                         const void* R, int64_t ldr, aic_dtype ab_type, aic_dtype c_type, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(r2 > 0, InvalidArgument, "gemm_lowrank: r2 must be positive");
        aic::hip::GemmArgs a;
        a.transA = transA;
        a.transB = transB;
        a.M = M;
        a.N = N;
        a.K = K;
        a.alpha = alpha;
        a.beta = beta;
        a.A = A;
        a.lda = lda;
        a.B = B;
        a.ldb = ldb;
        a.C = C;
        a.ldc = ldc;
        a.R = R;
        a.ldr = ldr;
        a.ab = dt(ab_type);
        a.c = dt(c_type);
        a.X2 = X2;
        a.ldx2 = ldx2;
        a.Y2 = Y2;
        a.ldy2 = ldy2;
        a.r2 = r2;
        a.seg_n = seg_n;
        a.y2_kmajor = y2_kmajor;
        aic::hip::gemm(a, st(stream));
    });
}

int aic_hip_rmsnorm_fwd(const void* x, int64_t ldx, const float* w, void* y, int64_t ldy, float* rms, int64_t rows,
                        int64_t dim, float eps, aic_dtype d, aic_stream stream) {
    return guard([&] { aic::hip::rmsnorm_fwd(x, ldx, w, y, ldy, rms, rows, dim, eps, dt(d), st(stream)); });
}

int aic_hip_rmsnorm_bwd(const void* dy, int64_t lddy, const void* x, int64_t ldx, const float* w, const float* rms,
                        const void* dres, int64_t ldres, void* dx, int64_t lddx, float* dw, int accumulate, int64_t rows,
                        int64_t dim, aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::rmsnorm_bwd(dy, lddy, x, ldx, w, rms, dres, ldres, dx, lddx, dw, accumulate != 0, rows, dim, dt(d),
                              st(stream));
    });
}

int aic_hip_rope(void* x, int64_t ld, int64_t B, int64_t S, int64_t heads, int64_t hd, int64_t start_pos,
                 const float* cos_t, const float* sin_t, int inverse, aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::rope(x, ld, B, S, heads, hd, start_pos, cos_t, sin_t, inverse != 0, dt(d), st(stream));
    });
}

int aic_hip_rope_tables(float* cos_host, float* sin_host, int64_t max_seq, int64_t hd, float base) {
    return guard([&] {
        AIC_CHECK(cos_host && sin_host && max_seq >= 0 && hd > 0 && hd % 2 == 0, InvalidArgument, "bad rope table args");
        aic::hip::rope_tables_host(cos_host, sin_host, max_seq, hd, base);
    });
}

int aic_hip_attn_fwd(const void* q, const void* k, const void* v, int64_t ld_qkv, void* o, int64_t ld_o, float* lse,
                     int64_t B, int64_t H, int64_t S, int64_t hd, int causal, float scale, aic_dtype d,
                     aic_stream stream) {
    return guard([&] {
        aic::hip::attn_fwd(q, k, v, ld_qkv, o, ld_o, lse, B, H, S, hd, causal != 0, scale, dt(d), st(stream));
    });
}

int aic_hip_attn_bwd(const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o, const void* dout,
                     int64_t ld_o, const float* lse, void* dq, void* dk, void* dv, int64_t ld_d, int64_t B, int64_t H,
                     int64_t S, int64_t hd, int causal, float scale, aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::attn_bwd(q, k, v, ld_qkv, o, dout, ld_o, lse, dq, dk, dv, ld_d, B, H, S, hd, causal != 0, scale,
                           dt(d), st(stream));
    });
}

int aic_hip_attn_fwd_qk(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_k, void* o, int64_t ld_o,
                        float* lse, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t hd, int causal, float scale,
                        aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::attn_fwd_qk(q, ld_q, k, v, ld_k, o, ld_o, lse, B, H, Sq, Sk, hd, causal != 0, scale, dt(d),
                              st(stream));
    });
}

int aic_hip_attn_bwd_qk(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_k, const void* o,
                        const void* dout, int64_t ld_o, const float* lse, void* dq, int64_t ld_dq, void* dk, void* dv,
                        int64_t ld_dkv, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t hd, int causal,
                        float scale, aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::attn_bwd_qk(q, ld_q, k, v, ld_k, o, dout, ld_o, lse, dq, ld_dq, dk, dv, ld_dkv, B, H, Sq, Sk, hd,
                              causal != 0, scale, dt(d), st(stream));
    });
}

int aic_hip_gemm_rope(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* W, int64_t ldw,
                      void* C, int64_t ldc, int64_t rope_cols, int64_t hd, int64_t seq, int64_t start_pos,
                      const float* cos_t, const float* sin_t, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(cos_t && sin_t, InvalidArgument, "gemm_rope: cos_t and sin_t are required");
        aic::hip::GemmArgs a;
        a.transA = 0;
        a.transB = 1;
        a.M = M;
        a.N = N;
        a.K = K;
        a.A = A;
        a.lda = lda;
        a.B = W;
        a.ldb = ldw;
        a.C = C;
        a.ldc = ldc;
        a.ab = aic::DType::BFloat16;
        a.c = aic::DType::BFloat16;
        a.rope_cos = cos_t;
        a.rope_sin = sin_t;
        a.rope_cols = rope_cols;
        a.rope_hd = hd;
        a.rope_seq = seq;
        a.rope_start = start_pos;
        aic::hip::gemm(a, st(stream));
    });
}

int aic_hip_gemm_swiglu(int64_t M, int64_t f, int64_t K, const void* A, int64_t lda, const void* W, int64_t ldw,
                        void* GU, int64_t ldgu, void* H, int64_t ldh, aic_stream stream) {
    return guard([&] {
        aic::hip::GemmArgs a;
        a.transA = 0;
        a.transB = 1;
        a.M = M;
        a.N = 2 * f;
        a.K = K;
        a.A = A;
        a.lda = lda;
        a.B = W;
        a.ldb = ldw;
        a.C = GU;
        a.ldc = ldgu;
        a.ab = aic::DType::BFloat16;
        a.c = aic::DType::BFloat16;
        a.glu_f = f;
        a.glu_out = H;
        a.ld_glu = ldh;
        aic::hip::gemm(a, st(stream));
    });
}

int aic_hip_lora_skinny(const void* Y, int64_t ldy, int64_t T, int64_t N, int64_t n_seg, int64_t r_seg, const void* W,
                        int64_t w_n, int64_t w_j, void* out1, int64_t ldo1, float scale, const void* Z, int64_t ldz,
                        float* out2, int64_t o2n, int64_t o2j, int accumulate, aic_stream stream) {
    return guard([&] {
        aic::hip::LoraSkinny q;
        q.Y = Y;
        q.ldy = ldy;
        q.T = T;
        q.N = N;
        q.n_seg = n_seg;
        q.r_seg = r_seg;
        q.W = W;
        q.w_n = w_n;
        q.w_j = w_j;
        q.out1 = out1;
        q.ldo1 = ldo1;
        q.scale = scale;
        q.Z = Z;
        q.ldz = ldz;
        q.out2 = out2;
        q.o2n = o2n;
        q.o2j = o2j;
        q.accumulate = accumulate != 0;
        AIC_CHECK(T >= 0 && N >= 0, InvalidArgument, "lora_skinny: negative size");
        if (T == 0 || N == 0) return;
        AIC_CHECK(aic::hip::lora_skinny_ok(q), NotImplemented, "lora_skinny: shape or layout outside the kernel's forms");
        aic::hip::lora_skinny(q, st(stream));
    });
}

int aic_hip_gemm_swiglu_bwd(int64_t M, int64_t f, int64_t K, const void* A, int64_t lda, const void* B, int64_t ldb,
                            const void* GU, int64_t ldgu, void* DH, int64_t lddh, void* DGU, aic_stream stream) {
    return guard([&] {
        aic::hip::GemmArgs a;
        a.transA = 0;
        a.transB = 0;
        a.M = M;
        a.N = f;
        a.K = K;
        a.A = A;
        a.lda = lda;
        a.B = B;
        a.ldb = ldb;
        a.C = DH;
        a.ldc = lddh;
        a.ab = aic::DType::BFloat16;
        a.c = aic::DType::BFloat16;
        a.dglu_gu = GU;
        a.dglu_out = DGU;
        a.dglu_ld = ldgu;
        aic::hip::gemm(a, st(stream));
    });
}

int aic_hip_attn_bwd_rope(const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o, const void* dout,
                          int64_t ld_o, const float* lse, void* dq, void* dk, void* dv, int64_t ld_d, int64_t B,
                          int64_t H, int64_t S, int64_t hd, int causal, float scale, const float* cos_t,
                          const float* sin_t, aic_dtype d, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(cos_t && sin_t, InvalidArgument, "attn_bwd_rope: cos_t and sin_t are required");
        aic::hip::attn_bwd(q, k, v, ld_qkv, o, dout, ld_o, lse, dq, dk, dv, ld_d, B, H, S, hd, causal != 0, scale,
                           dt(d), st(stream), cos_t, sin_t);
    });
}

int aic_hip_swiglu_fwd(const void* g, const void* u, int64_t ld_gu, void* h, int64_t ld_h, int64_t T, int64_t f,
                       aic_dtype d, aic_stream stream) {
    return guard([&] { aic::hip::swiglu_fwd(g, u, ld_gu, h, ld_h, T, f, dt(d), st(stream)); });
}

int aic_hip_swiglu_bwd(const void* g, const void* u, int64_t ld_gu, const void* dh, int64_t ld_h, void* dg, void* du,
                       int64_t ld_d, int64_t T, int64_t f, aic_dtype d, aic_stream stream) {
    return guard([&] { aic::hip::swiglu_bwd(g, u, ld_gu, dh, ld_h, dg, du, ld_d, T, f, dt(d), st(stream)); });
}

int aic_hip_ce_fwd(const void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
                   float* losses, float* lse, float* loss_mean, int64_t* valid, aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::ce_fwd(logits, ld, targets, N, C, ignore_index, losses, lse, loss_mean, valid, dt(d), st(stream));
    });
}

int aic_hip_ce_bwd(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                   int64_t ignore_index, const float* grad, const int64_t* valid, void* dlogits, int64_t ld_d,
                   aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::ce_bwd(logits, ld, targets, lse, N, C, ignore_index, grad, valid, dlogits, ld_d, dt(d), st(stream));
    });
}

int aic_hip_ce_fwd_bwd(void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
                       float* losses, float* lse, float* loss_mean, int64_t* valid, const float* grad, aic_dtype d,
                       aic_stream stream) {
    return guard([&] {
        aic::hip::ce_fwd_bwd(logits, ld, targets, N, C, ignore_index, losses, lse, loss_mean, valid, grad, dt(d),
                             st(stream));
    });
}

int aic_hip_ce_bwd_rows(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N,
                        int64_t C, int64_t ignore_index, const float* grad, int per_row, float divisor, void* dlogits,
                        int64_t ld_d, aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::ce_bwd_rows(logits, ld, targets, lse, N, C, ignore_index, grad, per_row, divisor, dlogits, ld_d,
                              dt(d), st(stream));
    });
}

int aic_hip_ce_fwd_soft(const void* logits, int64_t ld, const float* y, int64_t ld_y, int64_t N, int64_t C,
                        float* losses, float* lse, float* loss_mean, aic_dtype d, aic_stream stream) {
    return guard([&] { aic::hip::ce_fwd_soft(logits, ld, y, ld_y, N, C, losses, lse, loss_mean, dt(d), st(stream)); });
}

int aic_hip_ce_bwd_soft(const void* logits, int64_t ld, const float* y, int64_t ld_y, const float* lse, int64_t N,
                        int64_t C, const float* grad, int per_row, float divisor, void* dlogits, int64_t ld_d,
                        aic_dtype d, aic_stream stream) {
    return guard([&] {
        aic::hip::ce_bwd_soft(logits, ld, y, ld_y, lse, N, C, grad, per_row, divisor, dlogits, ld_d, dt(d),
                              st(stream));
    });
}

int aic_hip_memcpy_sync(void* dst, const void* src, size_t bytes, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(bytes == 0 || (dst && src), InvalidArgument, "memcpy_sync: null pointer");
        if (bytes == 0) return;
        AIC_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, st(stream)));
        AIC_HIP_CHECK(hipStreamSynchronize(st(stream)));
    });
}

int aic_hip_embed_fwd(const int64_t* ids, int64_t N, const void* W, int64_t V, int64_t D, void* out, aic_dtype d,
                      aic_stream stream) {
    return guard([&] { aic::hip::embed_fwd(ids, N, W, V, D, out, dt(d), st(stream)); });
}

int aic_hip_embed_bwd(const int64_t* ids, int64_t N, const void* dout, int64_t V, int64_t D, float* dW, int accumulate,
                      aic_dtype d, aic_stream stream) {
    return guard([&] { aic::hip::embed_bwd(ids, N, dout, V, D, dW, accumulate != 0, dt(d), st(stream)); });
}

int aic_hip_grad_sqnorm_multi(const float* const* grads, const int64_t* sizes, int count, double* sqnorm,
                              int* nonfinite, aic_stream stream) {
    return guard([&] { aic::hip::grad_sqnorm_multi(grads, sizes, count, sqnorm, nonfinite, st(stream)); });
}

int aic_hip_grad_sqnorm_multi_noalloc(const float* const* grads, const int64_t* sizes, int count, double* sqnorm,
                                      int* nonfinite, aic_stream stream) {
    return guard([&] { aic::hip::grad_sqnorm_multi_noalloc(grads, sizes, count, sqnorm, nonfinite, st(stream)); });
}

int aic_hip_scale_multi(float* const* grads, const int64_t* sizes, int count, const float* scale, aic_stream stream) {
    return guard([&] { aic::hip::scale_multi(grads, sizes, count, scale, st(stream)); });
}

int aic_hip_optim_finalize(const double* sqnorm, const int* nonfinite, aic_optim_ctl* ctl, aic_stream stream) {
    return guard([&] { aic::hip::optim_finalize(sqnorm, nonfinite, ctl, st(stream)); });
}

int aic_hip_adamw_multi(float* const* p, const float* const* g, float* const* m, float* const* v, void* const* p_bf16,
                        const int64_t* sizes, int count, float lr, float beta1, float beta2, float eps,
                        float weight_decay, int64_t step, const aic_optim_ctl* ctl, aic_stream stream) {
    return guard([&] {
        aic::hip::adamw_multi(p, g, m, v, p_bf16, sizes, count, lr, beta1, beta2, eps, weight_decay, step, ctl,
                              st(stream));
    });
}

int aic_hip_adamw_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                       float eps, float weight_decay, float bias_correction1, float bias_correction2,
                       aic_stream stream) {
    return guard([&] {
        aic::hip::adamw_step(p, g, m, v, n, lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2,
                             st(stream));
    });
}

int aic_hip_cast_f32_bf16(const float* src, void* dst, int64_t n, aic_stream stream) {
    return guard([&] { aic::hip::cast_f32_bf16(src, dst, n, st(stream)); });
}

int aic_hip_stream_probe(const float* const* in, int n_in, float* const* out, int n_out, void* out_bf16, float* sink,
                         int64_t n, int nontemporal, aic_stream stream) {
    return guard([&] { aic::hip::stream_probe(in, n_in, out, n_out, out_bf16, sink, n, nontemporal != 0, st(stream)); });
}

// ------------------------------------------------------------------ TransformerLM
int aic_lm_create(const aic_lm_config* cfg, const aic_train_config* tcfg, aic_lm** out) {
    return guard([&] {
        AIC_CHECK(cfg && tcfg && out, InvalidArgument, "null argument");
        aic::models::TransformerLMConfig c;
        c.vocab_size = cfg->vocab;
        c.hidden_dim = cfg->d_model;
        c.num_layers = cfg->n_layers;
        c.num_heads = cfg->n_heads;
        c.intermediate_dim = cfg->d_ffn;
        c.max_seq_len = cfg->max_seq_len;
        c.rms_norm_eps = cfg->norm_eps;
        c.rope_theta = cfg->rope_base;
        c.tie_word_embeddings = cfg->tied != 0;
        c.compute = dt(cfg->compute);
        c.num_experts = cfg->n_experts;
        c.top_k = cfg->top_k;
        c.aux_loss_coef = cfg->aux_loss_coef;
        c.lora_rank = cfg->lora_rank;
        c.lora_alpha = cfg->lora_alpha;
        c.quant_group = cfg->quant_group;
        aic::models::TrainOptions o;
        o.adamw = {tcfg->lr, tcfg->beta1, tcfg->beta2, tcfg->eps, tcfg->weight_decay};
        o.max_grad_norm = tcfg->max_grad_norm;
        o.use_loss_scaler = tcfg->use_loss_scaler != 0;
        o.scaler = {tcfg->init_scale, tcfg->growth_factor, tcfg->backoff_factor, tcfg->growth_interval,
                    tcfg->min_scale, tcfg->max_scale};
        auto* h = new aic_lm{nullptr};
        try {
            h->model = new aic::models::TransformerLM(c, o);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int aic_lm_destroy(aic_lm* lm) {
    return guard([&] {
        if (!lm) return;
        delete lm->model;
        delete lm;
    });
}

int64_t aic_lm_num_params(const aic_lm* lm) { return lm ? lm->model->num_params() : -1; }

int aic_lm_num_tensors(const aic_lm* lm) { return lm ? static_cast<int>(lm->model->params().size()) : -1; }

namespace {
int tensor_info(const std::vector<aic::models::ParamInfo>& ps, int i, char* name, int name_cap, int* rank,
                int64_t* dims, int64_t* offset) {
    return guard([&] {
        AIC_CHECK(i >= 0 && i < static_cast<int>(ps.size()), OutOfRange, "tensor index ", i);
        const auto& p = ps[static_cast<size_t>(i)];
        if (name && name_cap > 0) {
            std::strncpy(name, p.name.c_str(), static_cast<size_t>(name_cap) - 1);
            name[name_cap - 1] = '\0';
        }
        if (rank) *rank = static_cast<int>(p.shape.size());
        if (dims)
            for (size_t k = 0; k < p.shape.size() && k < 2; ++k) dims[k] = p.shape[k];
        if (offset) {
            int64_t o = 0;
            for (int j = 0; j < i; ++j) o += ps[static_cast<size_t>(j)].numel;
            *offset = o;  // offset in the packed (unpadded) host layout
        }
    });
}
}  // namespace

int aic_lm_tensor_info(const aic_lm* lm, int i, char* name, int name_cap, int* rank, int64_t* dims, int64_t* offset) {
    if (!lm) return guard([] { AIC_CHECK(false, InvalidArgument, "null model"); });
    return tensor_info(lm->model->params(), i, name, name_cap, rank, dims, offset);
}

int64_t aic_lm_num_base_params(const aic_lm* lm) {
    if (!lm) return -1;
    int64_t n = 0;
    for (const auto& p : lm->model->base_params()) n += p.numel;
    return n;
}

int aic_lm_num_base_tensors(const aic_lm* lm) {
    return lm ? static_cast<int>(lm->model->base_params().size()) : -1;
}

int aic_lm_base_tensor_info(const aic_lm* lm, int i, char* name, int name_cap, int* rank, int64_t* dims,
                            int64_t* offset) {
    if (!lm) return guard([] { AIC_CHECK(false, InvalidArgument, "null model"); });
    return tensor_info(lm->model->base_params(), i, name, name_cap, rank, dims, offset);
}

int aic_lm_set_base_params(aic_lm* lm, const float* host) {
    return guard([&] {
        AIC_CHECK(lm && host, InvalidArgument, "null argument");
        lm->model->set_base_params(host);
    });
}

int aic_lm_get_base_params(const aic_lm* lm, float* host) {
    return guard([&] {
        AIC_CHECK(lm && host, InvalidArgument, "null argument");
        lm->model->get_base_params(host);
    });
}

int aic_lm_set_params(aic_lm* lm, const float* host) { return guard([&] { lm->model->set_params(host); }); }
int aic_lm_get_params(const aic_lm* lm, float* host) { return guard([&] { lm->model->get_params(host); }); }
int aic_lm_get_grads(const aic_lm* lm, float* host) { return guard([&] { lm->model->get_grads(host); }); }
int aic_lm_moe_routing(const aic_lm* lm, int64_t layer, int64_t* idx_host, int64_t capacity, int64_t* tokens) {
    return guard([&] {
        AIC_CHECK(lm && tokens, InvalidArgument, "null argument");
        *tokens = lm->model->moe_routing(layer, idx_host, capacity);
    });
}
int aic_lm_get_adam_state(const aic_lm* lm, float* m, float* v, int64_t* step) {
    return guard([&] { lm->model->get_adam_state(m, v, step); });
}

int aic_lm_init_normal(aic_lm* lm, uint64_t seed, float std, int residual_scaling) {
    return guard([&] { lm->model->init_normal(seed, std, residual_scaling != 0); });
}

namespace {
struct IdsOnDevice {
    const int64_t* ids = nullptr;
    const int64_t* tgt = nullptr;
    aic::DeviceBuffer buf;
    IdsOnDevice(const int64_t* i, const int64_t* t, int64_t n, int on_device, hipStream_t s) {
        if (on_device) {
            ids = i;
            tgt = t;
            return;
        }
        buf = aic::DeviceBuffer(sizeof(int64_t) * 2 * static_cast<size_t>(n), s);
        int64_t* d = buf.as<int64_t>();
        AIC_HIP_CHECK(hipMemcpyAsync(d, i, sizeof(int64_t) * n, hipMemcpyHostToDevice, s));
        AIC_HIP_CHECK(hipMemcpyAsync(d + n, t, sizeof(int64_t) * n, hipMemcpyHostToDevice, s));
        AIC_HIP_CHECK(hipStreamSynchronize(s));
        ids = d;
        tgt = d + n;
    }
};

void fill_stats(const aic::models::StepStats& s, aic_step_stats* out) {
    out->loss = s.loss;
    out->grad_norm = s.grad_norm;
    out->found_inf = s.found_inf ? 1 : 0;
    out->loss_scale = s.loss_scale;
    out->step = s.step;
    out->aux_loss = s.aux_loss;
}
}  // namespace

int aic_lm_train_step(aic_lm* lm, const int64_t* ids, const int64_t* targets, int64_t B, int64_t S, int on_device,
                      aic_step_stats* stats) {
    return guard([&] {
        AIC_CHECK(lm && ids && targets, InvalidArgument, "null argument");
        IdsOnDevice in(ids, targets, B * S, on_device, lm->model->stream());
        lm->model->train_step(in.ids, in.tgt, B, S);
        if (stats) fill_stats(lm->model->last_stats(), stats);
    });
}

int aic_lm_eval_loss(aic_lm* lm, const int64_t* ids, const int64_t* targets, int64_t B, int64_t S, int on_device,
                     float* loss) {
    return guard([&] {
        AIC_CHECK(lm && ids && targets && loss, InvalidArgument, "null argument");
        IdsOnDevice in(ids, targets, B * S, on_device, lm->model->stream());
        *loss = lm->model->eval_loss(in.ids, in.tgt, B, S);
    });
}

int aic_lm_stream(const aic_lm* lm, aic_stream* stream) {
    return guard([&] { *stream = static_cast<aic_stream>(lm->model->stream()); });
}

int aic_lm_synchronize(aic_lm* lm) { return guard([&] { lm->model->synchronize(); }); }

int aic_lm_last_stats(aic_lm* lm, aic_step_stats* stats) {
    return guard([&] { fill_stats(lm->model->last_stats(), stats); });
}

int aic_lm_profile(aic_lm* lm, int enable) {
    return guard([&] {
        AIC_CHECK(lm, InvalidArgument, "null model");
        lm->model->set_profiling(enable != 0);
    });
}

int aic_lm_fused_grad_norm(aic_lm* lm, int enable, int* used) {
    return guard([&] {
        AIC_CHECK(lm, InvalidArgument, "null model");
        const bool u = lm->model->set_fused_grad_norm(enable != 0);
        if (used) *used = u ? 1 : 0;
    });
}

int aic_lm_profile_classes(aic_lm* lm, uint32_t class_mask) {
    return guard([&] {
        AIC_CHECK(lm, InvalidArgument, "null model");
        lm->model->set_profiling(class_mask != 0, class_mask);
    });
}

int aic_lm_profile_class_index(const char* name) { return aic::Profiler::class_index(name); }

int aic_lm_profile_stats(aic_lm* lm, aic_kernel_stat* out, int cap, int* n) {
    return guard([&] {
        AIC_CHECK(lm && n, InvalidArgument, "null argument");
        const auto st = lm->model->profile_stats();
        int k = 0;
        for (const auto& c : st) {
            if (k >= cap || !out) break;
            aic_kernel_stat& o = out[k++];
            std::memset(&o, 0, sizeof(o));
            std::strncpy(o.name, c.name.c_str(), sizeof(o.name) - 1);
            o.launches = c.launches;
            o.total_ms = c.total_ms;
            o.flops = c.flops;
            o.bytes = c.bytes;
            o.mfma_bound = c.mfma_bound ? 1 : 0;
        }
        *n = out ? k : static_cast<int>(st.size());
    });
}

// ------------------------------------------------------------------ synthetic data
int aic_synth_uniform_ids(uint64_t seed, int64_t n, int64_t vocab, int64_t* out_host) {
    return guard([&] {
        AIC_CHECK(out_host && n >= 0 && vocab > 0, InvalidArgument, "bad arguments");
        aic::data::uniform_ids(seed, n, vocab, out_host);
    });
}

int aic_synth_zipf_ids(uint64_t seed, int64_t n, int64_t vocab, double s, int64_t* out_host) {
    return guard([&] {
        AIC_CHECK(out_host && n >= 0 && vocab > 0 && s > 0, InvalidArgument, "bad arguments");
        aic::data::zipf_ids(seed, n, vocab, s, out_host);
    });
}

int aic_synth_normal(uint64_t seed, int64_t n, float mean, float std, float* out_host) {
    return guard([&] {
        AIC_CHECK(out_host && n >= 0, InvalidArgument, "bad arguments");
        aic::data::normal(seed, n, mean, std, out_host);
    });
}


// ---------------------------------------------------------------------------------------
// Mixture of experts
// ---------------------------------------------------------------------------------------
int aic_hip_moe_route(const float* logits, int64_t T, int64_t E, int64_t k, float aux_coef, int64_t* idx, float* gsel,
                      float* probs, float* rweights, int64_t* counts, float* mean_probs, float* aux, aic_stream stream) {
    return guard([&] {
        aic::hip::moe_route(logits, T, E, k, aux_coef, idx, gsel, probs, rweights, counts, mean_probs, aux, st(stream));
    });
}

int64_t aic_hip_moe_max_rows(int64_t T, int64_t E, int64_t k) { return aic::hip::moe_max_rows(T, E, k); }

int aic_hip_moe_permute(const int64_t* idx, const int64_t* counts, int64_t T, int64_t k, int64_t E, int64_t* offsets,
                        int32_t* dst_row, int32_t* src_ent, aic_stream stream) {
    return guard([&] { aic::hip::moe_permute(idx, counts, T, k, E, offsets, dst_row, src_ent, st(stream)); });
}

int aic_hip_moe_gather(const void* x, int64_t ldx, const int32_t* src_ent, int64_t k, int64_t rows, int64_t d,
                       void* xp, aic_dtype dtype, aic_stream stream) {
    return guard([&] { aic::hip::moe_gather(x, ldx, src_ent, k, rows, d, xp, dt(dtype), st(stream)); });
}

int aic_hip_moe_combine(const void* ye, const int64_t* idx, const int32_t* dst_row, const float* gsel, int64_t T,
                        int64_t k, int64_t d, const void* residual, int64_t ldr, void* out, int64_t ldo, aic_dtype dtype,
                        aic_stream stream) {
    return guard([&] {
        aic::hip::moe_combine(ye, idx, dst_row, gsel, T, k, d, residual, ldr, out, ldo, dt(dtype), st(stream));
    });
}

int aic_moe_ffn_create(int64_t d_model, int64_t d_hidden, int64_t num_experts, int64_t top_k, float aux_loss_coef,
                       aic_dtype dtype, aic_moe_ffn** out) {
    return guard([&] {
        AIC_CHECK(out, InvalidArgument, "null argument");
        auto* h = new aic_moe_ffn{nullptr};
        try {
            h->ffn = new aic::models::MoEFFN(d_model, d_hidden, num_experts, top_k, aux_loss_coef, dt(dtype));
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int aic_moe_ffn_destroy(aic_moe_ffn* m) {
    return guard([&] {
        if (!m) return;
        delete m->ffn;
        delete m;
    });
}

int aic_moe_ffn_forward(aic_moe_ffn* m, const void* h, int64_t T, const void* router_w, const void* experts,
                        const void* residual, void* y, float* aux, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(m, InvalidArgument, "null handle");
        m->ffn->forward(h, T, router_w, experts, residual, y, aux, st(stream));
    });
}

int aic_moe_ffn_backward(aic_moe_ffn* m, const void* dy, float daux, void* dh, float* drouter_w, float* dexperts,
                         aic_stream stream) {
    return guard([&] {
        AIC_CHECK(m, InvalidArgument, "null handle");
        m->ffn->backward(dy, daux, dh, drouter_w, dexperts, st(stream));
    });
}

int aic_moe_ffn_routing(aic_moe_ffn* m, int64_t* idx_host, int64_t* counts_host, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(m && idx_host && counts_host, InvalidArgument, "null argument");
        (void)stream;
        AIC_HIP_CHECK(hipDeviceSynchronize());
        const auto& ch = m->ffn->counts_host();
        int64_t T = 0;
        for (size_t e = 0; e < ch.size(); ++e) {
            counts_host[e] = ch[e];
            T += ch[e];
        }
        AIC_HIP_CHECK(hipMemcpy(idx_host, m->ffn->idx(), sizeof(int64_t) * T, hipMemcpyDeviceToHost));
    });
}

// ------------------------------------------------------------------ INT4 + LoRA
int aic_hip_int4_quantize(const float* x, int64_t n, int64_t group, uint8_t* packed, void* scales,
                          aic_dtype scale_type, aic_stream stream) {
    return guard([&] { aic::hip::int4_quantize(x, n, group, packed, scales, dt(scale_type), st(stream)); });
}

int aic_hip_int4_dequantize(const uint8_t* packed, const void* scales, aic_dtype scale_type, int64_t n, int64_t group,
                            void* out, aic_dtype out_type, aic_stream stream) {
    return guard([&] { aic::hip::int4_dequant(packed, scales, dt(scale_type), n, group, out, dt(out_type), st(stream)); });
}

int aic_hip_int4_dequantize_zp(const uint8_t* packed, const float* scales, const float* zero_points, int is_signed,
                               int64_t n, int64_t group, float* out, aic_stream stream) {
    return guard([&] { aic::hip::int4_dequant_zp(packed, scales, zero_points, is_signed != 0, n, group, out, st(stream)); });
}

int aic_hip_int4_dequant_gemm(int transW, int64_t M, int64_t N, int64_t K, float alpha, const void* X, int64_t ldx,
                              const uint8_t* Wq, const void* scales, aic_dtype scale_type, int64_t group, float beta,
                              void* C, int64_t ldc, const void* R, int64_t ldr, aic_dtype ab_type, aic_dtype c_type,
                              aic_stream stream) {
    return guard([&] {
        aic::models::int4_dequant_gemm(transW, M, N, K, alpha, X, ldx, Wq, scales, dt(scale_type), group, beta, C, ldc,
                                       R, ldr, dt(ab_type), dt(c_type), st(stream));
    });
}

int aic_hip_int4_gemm_swiglu(int64_t M, int64_t f, int64_t K, const void* X, int64_t ldx, const uint8_t* Wq,
                             const void* scales, int64_t group, const void* X2, int64_t ldx2, const void* Y2,
                             int64_t ldy2, int64_t r2, int64_t seg_n, void* GU, int64_t ldgu, void* H, int64_t ldh,
                             aic_stream stream) {
    return guard([&] {
        AIC_CHECK(r2 >= 0 && (r2 == 0 || (X2 && Y2)) && H && f > 0, InvalidArgument,
                  "int4_gemm_swiglu: bad arguments");
        aic::hip::GemmArgs a;
        a.transA = 0;
        a.transB = 1;
        a.M = M;
        a.N = 2 * f;
        a.K = K;
        a.A = X;
        a.lda = ldx;
        a.ldb = K;
        a.Bq = Wq;
        a.Bscale = scales;
        a.scale_t = aic::DType::Float16;
        a.group = aic::hip::int4_group(2 * f * K, group);
        a.C = GU;
        a.ldc = ldgu;
        a.ab = aic::DType::BFloat16;
        a.c = aic::DType::BFloat16;
        if (r2 > 0) {
            a.X2 = X2;
            a.ldx2 = ldx2;
            a.Y2 = Y2;
            a.ldy2 = ldy2;
            a.r2 = r2;
            a.seg_n = seg_n;
        }
        a.glu_f = f;
        a.glu_out = H;
        a.ld_glu = ldh;
        const bool tiles = M % 256 == 0 && (2 * f) % 256 == 0 && f % 128 == 0 && (M / 256) * (2 * f / 256) >= 128;
        AIC_CHECK(tiles && aic::hip::gemm_q4_eligible(a) &&
                      (r2 == 0 || (r2 % 8 == 0 && ldx2 % 8 == 0 && ldy2 % 8 == 0 && (seg_n == 0 || seg_n % 256 == 0))),
                  NotImplemented, "int4_gemm_swiglu: shape outside the INT4 GEMM's SwiGLU epilogue");
        aic::hip::gemm(a, st(stream));
    });
}

int aic_hip_int4_gemm_rope(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, const uint8_t* Wq,
                           const void* scales, int64_t group, const void* X2, int64_t ldx2, const void* Y2, int64_t ldy2,
                           int64_t r2, int64_t seg_n, void* C, int64_t ldc, int64_t rope_cols, int64_t hd, int64_t seq,
                           int64_t start_pos, const float* cos_t, const float* sin_t, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(cos_t && sin_t, InvalidArgument, "int4_gemm_rope: cos_t and sin_t are required");
        AIC_CHECK(r2 >= 0 && (r2 == 0 || (X2 && Y2)), InvalidArgument, "int4_gemm_rope: bad low-rank term");
        aic::hip::GemmArgs a;
        a.transA = 0;
        a.transB = 1;
        a.M = M;
        a.N = N;
        a.K = K;
        a.A = X;
        a.lda = ldx;
        a.ldb = K;
        a.Bq = Wq;
        a.Bscale = scales;
        a.scale_t = aic::DType::Float16;
        a.group = group;
        a.C = C;
        a.ldc = ldc;
        a.ab = aic::DType::BFloat16;
        a.c = aic::DType::BFloat16;
        if (r2 > 0) {
            a.X2 = X2;
            a.ldx2 = ldx2;
            a.Y2 = Y2;
            a.ldy2 = ldy2;
            a.r2 = r2;
            a.seg_n = seg_n;
        }
        a.rope_cos = cos_t;
        a.rope_sin = sin_t;
        a.rope_cols = rope_cols;
        a.rope_hd = hd;
        a.rope_seq = seq;
        a.rope_start = start_pos;
        aic::hip::gemm(a, st(stream));
    });
}

int aic_hip_lora_merge(void* W, const void* A, const void* B, int64_t in_features, int64_t out_features, int64_t rank,
                       float scaling, int sign, aic_dtype dtype, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(W && A && B && in_features > 0 && out_features > 0 && rank > 0, InvalidArgument, "bad lora_merge args");
        aic::hip::GemmArgs a;
        a.M = out_features;
        a.N = in_features;
        a.K = rank;
        a.alpha = sign >= 0 ? scaling : -scaling;
        a.A = B;
        a.lda = rank;
        a.B = A;
        a.ldb = in_features;
        a.beta = 1.0f;
        a.C = W;
        a.ldc = in_features;
        a.ab = dt(dtype);
        a.c = dt(dtype);
        aic::hip::gemm(a, st(stream));
    });
}

int aic_qlora_linear_create(int64_t in_features, int64_t out_features, int64_t rank, float alpha, int64_t group,
                            aic_dtype scale_type, aic_dtype dtype, aic_qlora_linear** out) {
    return guard([&] {
        AIC_CHECK(out, InvalidArgument, "null argument");
        auto* h = new aic_qlora_linear{nullptr};
        try {
            h->lin = new aic::models::QLoRALinear(in_features, out_features, rank, alpha, group, dt(scale_type), dt(dtype));
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int aic_qlora_linear_destroy(aic_qlora_linear* m) {
    return guard([&] {
        if (!m) return;
        delete m->lin;
        delete m;
    });
}

int aic_qlora_linear_forward(aic_qlora_linear* m, const void* x, int64_t T, const uint8_t* Wq, const void* scales,
                             const void* A, const void* B, const void* R, void* y, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(m, InvalidArgument, "null module");
        m->lin->forward(x, T, Wq, scales, A, B, R, y, st(stream));
    });
}

int aic_qlora_linear_backward(aic_qlora_linear* m, const void* dy, void* dx, float* dA, float* dB, int accumulate,
                              aic_stream stream) {
    return guard([&] {
        AIC_CHECK(m, InvalidArgument, "null module");
        m->lin->backward(dy, dx, dA, dB, accumulate != 0, st(stream));
    });
}

// ------------------------------------------------------------------ tensor primitives
int aic_hip_strided_copy(const void* src, int64_t offset, int ndim, const int64_t* shape, const int64_t* strides,
                         int64_t elem_size, void* dst, aic_stream stream) {
    return guard([&] { aic::hip::strided_copy(src, offset, ndim, shape, strides, elem_size, dst, st(stream)); });
}

int aic_hip_cast(const void* src, aic_dtype from, void* dst, aic_dtype to, int64_t n, aic_stream stream) {
    return guard([&] { aic::hip::cast(src, dt(from), dst, dt(to), n, st(stream)); });
}

int aic_hip_binary(int op, const float* a, int64_t a_offset, int a_ndim, const int64_t* a_shape,
                   const int64_t* a_strides, const float* b, int64_t b_offset, int b_ndim, const int64_t* b_shape,
                   const int64_t* b_strides, float* out, aic_stream stream) {
    return guard([&] {
        aic::hip::binary(op, a, a_offset, a_ndim, a_shape, a_strides, b, b_offset, b_ndim, b_shape, b_strides, out,
                         st(stream));
    });
}

int aic_hip_unary(int op, const float* x, float* y, int64_t n, aic_stream stream) {
    return guard([&] { aic::hip::unary(op, x, y, n, st(stream)); });
}

int aic_hip_reduce_all(int op, const float* x, int64_t n, float* out, aic_stream stream) {
    return guard([&] { aic::hip::reduce_all(op, x, n, out, st(stream)); });
}

int aic_hip_reduce_dim(int op, const float* x, int ndim, const int64_t* shape, int dim, float* out, aic_stream stream) {
    return guard([&] { aic::hip::reduce_dim(op, x, ndim, shape, dim, out, st(stream)); });
}

int aic_hip_cat(const void* const* srcs, const int64_t* mids, int count, int64_t outer, int64_t inner,
                int64_t elem_size, void* dst, aic_stream stream) {
    return guard([&] { aic::hip::cat(srcs, mids, count, outer, inner, elem_size, dst, st(stream)); });
}

int aic_hip_sum_to_shape(const float* grad, int ndim, const int64_t* shape, int target_ndim,
                         const int64_t* target_shape, float* out, aic_stream stream) {
    return guard([&] { aic::hip::sum_to_shape(grad, ndim, shape, target_ndim, target_shape, out, st(stream)); });
}

}  // extern "C"

int aic_checkpoint_write(const char* path, int64_t step, int64_t epoch, float best_val_loss, const char* description,
                         int64_t n, const char* const* names, const int32_t* ranks, const int64_t* dims,
                         const int32_t* dtypes, const void* const* data, const uint64_t* nbytes) {
    return guard([&] {
        AIC_CHECK(path && n >= 0 && (n == 0 || (names && ranks && dtypes && data && nbytes)), InvalidArgument,
                  "aic_checkpoint_write: null argument");
        aic::CheckpointMeta meta{step, epoch, best_val_loss, description ? description : ""};
        std::vector<aic::CheckpointTensorRef> refs;
        const int64_t* d = dims;
        for (int64_t i = 0; i < n; ++i) {
            AIC_CHECK(names[i] && ranks[i] >= 0 && (ranks[i] == 0 || d), InvalidArgument,
                      "aic_checkpoint_write: bad tensor ", i);
            std::vector<int64_t> shape(d, d + ranks[i]);
            d += ranks[i];
            refs.push_back({names[i], shape, dtypes[i], data[i], nbytes[i]});
        }
        aic::write_checkpoint(path, meta, refs);
    });
}

int aic_checkpoint_verify(const char* path, int64_t* num_tensors, int64_t* step, int64_t* epoch, float* best_val_loss) {
    return guard([&] {
        AIC_CHECK(path, InvalidArgument, "aic_checkpoint_verify: null path");
        aic::CheckpointMeta meta;
        std::vector<aic::CheckpointTensor> ts;
        aic::read_checkpoint(path, meta, ts);
        if (num_tensors) *num_tensors = static_cast<int64_t>(ts.size());
        if (step) *step = meta.step;
        if (epoch) *epoch = meta.epoch;
        if (best_val_loss) *best_val_loss = meta.best_val_loss;
    });
}

int aic_checkpoint_module_order(int64_t n, const char* const* names, int64_t* order) {
    return guard([&] {
        AIC_CHECK(n >= 0 && (n == 0 || (names && order)), InvalidArgument, "aic_checkpoint_module_order: null argument");
        std::vector<std::string> v;
        for (int64_t i = 0; i < n; ++i) {
            AIC_CHECK(names[i], InvalidArgument, "aic_checkpoint_module_order: null name ", i);
            v.emplace_back(names[i]);
        }
        const std::vector<size_t> idx = aic::module_order(v);
        for (int64_t i = 0; i < n; ++i) order[i] = static_cast<int64_t>(idx[static_cast<size_t>(i)]);
    });
}

int aic_lm_save_checkpoint(aic_lm* lm, const char* path, int64_t step, int64_t epoch, float best_val_loss,
                           const char* description, int with_optimizer) {
    return guard([&] {
        AIC_CHECK(lm && path, InvalidArgument, "null argument");
        aic::CheckpointMeta meta{step, epoch, best_val_loss, description ? description : ""};
        lm->model->save_checkpoint(path, meta, with_optimizer != 0);
    });
}

int aic_lm_load_checkpoint(aic_lm* lm, const char* path, int64_t* step, int64_t* epoch, float* best_val_loss,
                           char* description, int desc_cap, int* has_optimizer) {
    return guard([&] {
        AIC_CHECK(lm && path, InvalidArgument, "null argument");
        bool has = false;
        const aic::CheckpointMeta meta = lm->model->load_checkpoint(path, &has);
        if (step) *step = meta.step;
        if (epoch) *epoch = meta.epoch;
        if (best_val_loss) *best_val_loss = meta.best_val_loss;
        if (description && desc_cap > 0) {
            std::strncpy(description, meta.description.c_str(), static_cast<size_t>(desc_cap) - 1);
            description[desc_cap - 1] = '\0';
        }
        if (has_optimizer) *has_optimizer = has ? 1 : 0;
    });
}

struct aic_token_dataset {
    std::shared_ptr<aic::data::TokenDataset> ds;
};
struct aic_token_loader {
    std::unique_ptr<aic::data::TokenLoader> loader;
};

int aic_dataset_open(const char* path, int64_t seq_len, int64_t stride, aic_token_dataset** out) {
    return guard([&] {
        AIC_CHECK(path && out, InvalidArgument, "null argument");
        *out = new aic_token_dataset{std::make_shared<aic::data::TokenDataset>(path, seq_len, stride)};
    });
}

int aic_dataset_from_tokens(const int64_t* tokens, int64_t n, int64_t seq_len, int64_t stride,
                            aic_token_dataset** out) {
    return guard([&] {
        AIC_CHECK(out && n >= 0 && (tokens || n == 0), InvalidArgument, "null argument");
        std::vector<int64_t> v(tokens, tokens + n);
        *out = new aic_token_dataset{std::make_shared<aic::data::TokenDataset>(std::move(v), seq_len, stride)};
    });
}

int aic_dataset_destroy(aic_token_dataset* ds) {
    return guard([&] { delete ds; });
}

int64_t aic_dataset_size(const aic_token_dataset* ds) { return ds ? ds->ds->size() : -1; }
int64_t aic_dataset_total_tokens(const aic_token_dataset* ds) { return ds ? ds->ds->total_tokens() : -1; }

int aic_dataset_get_item(const aic_token_dataset* ds, int64_t idx, int64_t* input, int64_t* target) {
    return guard([&] {
        AIC_CHECK(ds, InvalidArgument, "null dataset");
        ds->ds->get_item(idx, input, target);
    });
}

int aic_dataset_write_binary_file(const char* path, const int64_t* tokens, int64_t n) {
    return guard([&] {
        AIC_CHECK(path && n >= 0 && (tokens || n == 0), InvalidArgument, "null argument");
        aic::data::TokenDataset::write_binary_file(path, tokens, n);
    });
}

int aic_loader_create(aic_token_dataset* ds, int64_t batch_size, int shuffle, int drop_last, uint64_t seed,
                      int resident, aic_token_loader** out) {
    return guard([&] {
        AIC_CHECK(ds && out, InvalidArgument, "null argument");
        *out = new aic_token_loader{std::make_unique<aic::data::TokenLoader>(ds->ds, batch_size, shuffle != 0,
                                                                             drop_last != 0, seed, resident != 0)};
    });
}

int aic_loader_destroy(aic_token_loader* loader) {
    return guard([&] { delete loader; });
}

int64_t aic_loader_num_batches(const aic_token_loader* loader) { return loader ? loader->loader->num_batches() : -1; }
int aic_loader_has_next(const aic_token_loader* loader) { return loader && loader->loader->has_next() ? 1 : 0; }

int aic_loader_reset(aic_token_loader* loader) {
    return guard([&] {
        AIC_CHECK(loader, InvalidArgument, "null loader");
        loader->loader->reset();
    });
}

int aic_loader_next_host(aic_token_loader* loader, int64_t* inputs, int64_t* targets, int64_t* actual_batch) {
    return guard([&] {
        AIC_CHECK(loader && inputs && targets, InvalidArgument, "null argument");
        const int64_t b = loader->loader->next_host(inputs, targets);
        if (actual_batch) *actual_batch = b;
    });
}

int aic_loader_next_device(aic_token_loader* loader, int64_t* inputs, int64_t* targets, int64_t* actual_batch,
                           aic_stream stream) {
    return guard([&] {
        AIC_CHECK(loader && inputs && targets, InvalidArgument, "null argument");
        const int64_t b = loader->loader->next_device(inputs, targets, st(stream));
        if (actual_batch) *actual_batch = b;
    });
}

int aic_lm_forward_step(aic_lm* lm, const int64_t* ids, int64_t B, int64_t S, int64_t start_pos, int on_device,
                        float* logits) {
    return guard([&] {
        AIC_CHECK(lm && ids && logits && B > 0 && S > 0, InvalidArgument, "forward_step: bad arguments");
        auto* m = lm->model;
        hipStream_t s = m->stream();
        const int64_t V = m->config().vocab_size, T = B * S;
        if (on_device) {
            m->forward_step(ids, B, S, start_pos, logits);
            return;
        }
        aic::DeviceBuffer dids(sizeof(int64_t) * static_cast<size_t>(T), s), dl(sizeof(float) * T * V, s);
        AIC_HIP_CHECK(hipMemcpyAsync(dids.get(), ids, sizeof(int64_t) * T, hipMemcpyHostToDevice, s));
        m->forward_step(dids.as<int64_t>(), B, S, start_pos, dl.as<float>());
        AIC_HIP_CHECK(hipMemcpyAsync(logits, dl.get(), sizeof(float) * T * V, hipMemcpyDeviceToHost, s));
        AIC_HIP_CHECK(hipStreamSynchronize(s));
    });
}

int aic_sample_tokens(const float* logits, int64_t V, float temperature, int top_k, float top_p, uint64_t seed,
                      int64_t n_draws, int64_t* out) {
    return guard([&] {
        AIC_CHECK(logits && out && V > 0 && n_draws >= 0, InvalidArgument, "sample_tokens: bad arguments");
        const std::vector<float> l(logits, logits + V);
        std::mt19937_64 rng(seed);
        for (int64_t i = 0; i < n_draws; ++i) out[i] = aic::models::sample_token(l, temperature, top_k, top_p, rng);
    });
}

int aic_lm_generate(aic_lm* lm, const int64_t* prompt, int64_t n_prompt, int64_t max_new_tokens, float temperature,
                    int top_k, float top_p, int64_t eos_token_id, uint64_t seed, int64_t* out_tokens, int64_t* n_out) {
    return guard([&] {
        AIC_CHECK(lm && out_tokens && n_out && n_prompt >= 0 && (prompt || n_prompt == 0), InvalidArgument,
                  "generate: bad arguments");
        std::vector<int64_t> p(prompt, prompt + n_prompt);
        const std::vector<int64_t> out =
            lm->model->generate(p, max_new_tokens, temperature, top_k, top_p, eos_token_id, seed);
        std::copy(out.begin(), out.end(), out_tokens);
        *n_out = static_cast<int64_t>(out.size());
    });
}

int aic_lm_step_history(aic_lm* lm, aic_step_record* out, int cap, int* n, int64_t* dropped) {
    return guard([&] {
        AIC_CHECK(lm && n && (out || cap == 0), InvalidArgument, "null argument");
        *n = lm->model->step_history(out, cap, dropped);
    });
}

int aic_lm_snapshot(aic_lm* lm) {
    return guard([&] {
        AIC_CHECK(lm, InvalidArgument, "null model");
        lm->model->snapshot();
    });
}

int aic_lm_restore(aic_lm* lm) {
    return guard([&] {
        AIC_CHECK(lm, InvalidArgument, "null model");
        lm->model->restore();
    });
}

struct aic_telemetry {
    aic::TelemetryTracker t;
};

int aic_telemetry_create(int64_t window, float alpha_short, float alpha_long, aic_telemetry** out) {
    return guard([&] {
        AIC_CHECK(out && window > 0, InvalidArgument, "telemetry: bad arguments");
        *out = new aic_telemetry{aic::TelemetryTracker(static_cast<size_t>(window), alpha_short, alpha_long)};
    });
}

int aic_telemetry_destroy(aic_telemetry* t) {
    return guard([&] { delete t; });
}

int aic_telemetry_record(aic_telemetry* t, int64_t step, float loss, float grad_norm, float lr, float tokens_per_sec,
                         double step_seconds, int64_t total_tokens, int64_t model_params, int device_index,
                         aic_telemetry_snapshot* out) {
    return guard([&] {
        AIC_CHECK(t, InvalidArgument, "null tracker");
        const aic::TelemetrySnapshot s = t->t.record_step(step, loss, grad_norm, lr, tokens_per_sec, step_seconds,
                                                          total_tokens, model_params, device_index);
        if (out) {
            out->step = s.step;
            out->loss = s.loss;
            out->loss_ema_short = s.loss_ema_short;
            out->loss_ema_long = s.loss_ema_long;
            out->loss_variance = s.loss_variance;
            out->grad_norm = s.grad_norm;
            out->grad_norm_ema = s.grad_norm_ema;
            out->lr = s.lr;
            out->tokens_per_sec = s.tokens_per_sec;
            out->estimated_tflops = s.estimated_tflops;
            out->host_total_bytes = s.memory.host_total;
            out->host_free_bytes = s.memory.host_free;
            out->gpu_total_bytes = s.memory.gpu_total;
            out->gpu_free_bytes = s.memory.gpu_free;
            out->anomaly = static_cast<int32_t>(s.anomaly);
            out->pad = 0;
        }
    });
}

int64_t aic_telemetry_count(const aic_telemetry* t) { return t ? static_cast<int64_t>(t->t.count()) : -1; }
int aic_telemetry_is_nan_or_inf(const aic_telemetry* t) { return t && t->t.is_nan_or_inf() ? 1 : 0; }
int aic_telemetry_is_diverging(const aic_telemetry* t, float threshold_ratio, int min_consecutive) {
    return t && t->t.is_diverging(threshold_ratio > 0.0f ? threshold_ratio : 1.4f,
                                  min_consecutive > 0 ? min_consecutive : 3)
               ? 1
               : 0;
}
int aic_telemetry_is_gradient_exploding(const aic_telemetry* t, float spike_factor) {
    return t && t->t.is_gradient_exploding(spike_factor > 0.0f ? spike_factor : 4.0f) ? 1 : 0;
}
int aic_telemetry_is_gradient_vanishing(const aic_telemetry* t, float min_norm) {
    return t && t->t.is_gradient_vanishing(min_norm > 0.0f ? min_norm : 1e-7f) ? 1 : 0;
}
int aic_telemetry_reset(aic_telemetry* t) {
    return guard([&] {
        AIC_CHECK(t, InvalidArgument, "null tracker");
        t->t.reset();
    });
}
int aic_telemetry_latest_json(const aic_telemetry* t, char* buf, int cap) {
    return guard([&] {
        AIC_CHECK(t && buf && cap > 0, InvalidArgument, "null argument");
        const std::string j = t->t.latest().to_json();
        std::strncpy(buf, j.c_str(), static_cast<size_t>(cap) - 1);
        buf[cap - 1] = '\0';
    });
}

int aic_hip_gemm_ragged(int transB, int64_t M, int64_t N, int64_t K, float alpha, const void* A, int64_t lda,
                        const void* B, int64_t ldb, int64_t b_stride, void* C, int64_t ldc, const int64_t* offsets,
                        int E, int64_t glu_f, void* glu_out, int64_t ld_glu, const void* dglu_gu, void* dglu_out,
                        int64_t dglu_ld, aic_dtype c_type, aic_stream stream) {
    return guard([&] {
        aic::hip::RaggedArgs r;
        aic::hip::GemmArgs& a = r.g;
        a.transA = 0;
        a.transB = transB ? 1 : 0;
        a.M = M;
        a.N = N;
        a.K = K;
        a.alpha = alpha;
        a.A = A;
        a.lda = lda;
        a.B = B;
        a.ldb = ldb;
        a.C = C;
        a.ldc = ldc;
        a.ab = aic::DType::BFloat16;
        a.c = dt(c_type);
        a.glu_f = glu_f;
        a.glu_out = glu_out;
        a.ld_glu = ld_glu;
        a.dglu_gu = dglu_gu;
        a.dglu_out = dglu_out;
        a.dglu_ld = dglu_ld;
        r.offsets = offsets;
        r.E = E;
        r.b_stride = b_stride;
        AIC_CHECK(aic::hip::gemm_ragged_eligible(r), NotImplemented, "gemm_ragged: shape or layout not supported");
        aic::hip::gemm_ragged(r, st(stream));
    });
}

int aic_hip_gemm_grouped(int n, const aic_gemm_desc* descs, float alpha, float beta, aic_dtype ab_type,
                         aic_dtype c_type, aic_stream stream) {
    return guard([&] {
        AIC_CHECK(n >= 0 && (descs || n == 0), InvalidArgument, "gemm_grouped: bad arguments");
        std::vector<aic::hip::GemmArgs> v(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i) {
            const aic_gemm_desc& d = descs[i];
            aic::hip::GemmArgs& a = v[static_cast<size_t>(i)];
            a.transA = d.transA;
            a.transB = d.transB;
            a.M = d.M;
            a.N = d.N;
            a.K = d.K;
            a.A = d.A;
            a.lda = d.lda;
            a.B = d.B;
            a.ldb = d.ldb;
            a.C = d.C;
            a.ldc = d.ldc;
            a.alpha = alpha;
            a.beta = beta;
            a.ab = dt(ab_type);
            a.c = dt(c_type);
            AIC_CHECK(a.A && a.B && a.C && a.M >= 0 && a.N >= 0 && a.K >= 0, InvalidArgument,
                      "gemm_grouped: bad product ", i);
        }
        aic::hip::gemm_grouped(v.data(), n, st(stream));
    });
}
