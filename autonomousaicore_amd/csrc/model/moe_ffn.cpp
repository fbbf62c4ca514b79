#include "moe_ffn.hpp"

#include <algorithm>
#include <vector>

#include "../kernels/gemm.hpp"
#include "../kernels/kernels.hpp"
#include "../runtime/error.hpp"

namespace aic::models {

namespace {

void gemm(int ta, int tb, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* B, int64_t ldb,
          void* C, int64_t ldc, DType ab, DType c, hipStream_t s, float beta = 0.0f) {
    hip::GemmArgs a;
    a.transA = ta;
    a.transB = tb;
    a.M = M;
    a.N = N;
    a.K = K;
    a.A = A;
    a.lda = lda;
    a.B = B;
    a.ldb = ldb;
    a.C = C;
    a.ldc = ldc;
    a.beta = beta;
    a.ab = ab;
    a.c = c;
    hip::gemm(a, s);
}

hip::GemmArgs args(int ta, int tb, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* B,
                   int64_t ldb, void* C, int64_t ldc, DType ab, DType c) {
    hip::GemmArgs a;
    a.transA = ta;
    a.transB = tb;
    a.M = M;
    a.N = N;
    a.K = K;
    a.A = A;
    a.lda = lda;
    a.B = B;
    a.ldb = ldb;
    a.C = C;
    a.ldc = ldc;
    a.ab = ab;
    a.c = c;
    return a;
}

// The experts' products of one kind in launches of up to 8 (hip::gemm_grouped).
void run_grouped(const std::vector<hip::GemmArgs>& v, hipStream_t s) {
    for (size_t i = 0; i < v.size(); i += 8)
        hip::gemm_grouped(v.data() + i, static_cast<int>(std::min<size_t>(8, v.size() - i)), s);
}

}  // namespace

MoEFFN::MoEFFN(int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, DType dt)
    : d_(d), f_(f), E_(E), k_(k), coef_(aux_coef), dt_(dt) {
    AIC_CHECK(d > 0 && f > 0 && E >= 1 && E <= 64 && k >= 1 && k <= 8 && k <= E, InvalidArgument,
              "MoEFFN: need d, f > 0, 1 <= E <= 64, 1 <= top_k <= min(E, 8)");
    AIC_CHECK(dt == DType::Float32 || dt == DType::BFloat16, DTypeMismatch, "MoEFFN: dtype must be f32 or bf16");
}

void MoEFFN::forward(const void* h, int64_t T, const void* wr, const void* experts, const void* R, void* y,
                     float* aux, hipStream_t s) {
    AIC_CHECK(h && wr && experts && y && aux && T > 0, InvalidArgument, "MoEFFN::forward: bad arguments");
    const size_t es = dtype_size(dt_);
    const int64_t rows = hip::moe_max_rows(T, E_, k_), f2 = 2 * f_, ex = 3 * f_ * d_;
    T_ = T;
    h_ = h;
    wr_ = wr;
    ex_ = experts;
    logits_ = DeviceBuffer(sizeof(float) * T * E_, s);
    idx_ = DeviceBuffer(sizeof(int64_t) * T * k_, s);
    gsel_ = DeviceBuffer(sizeof(float) * T * k_, s);
    probs_ = DeviceBuffer(sizeof(float) * T * E_, s);
    counts_ = DeviceBuffer(sizeof(int64_t) * E_, s);
    offsets_ = DeviceBuffer(sizeof(int64_t) * (E_ + 1), s);
    dst_row_ = DeviceBuffer(sizeof(int) * T * k_, s);
    src_ent_ = DeviceBuffer(sizeof(int) * rows, s);
    // router logits in fp32, routing, dispatch order
    gemm(0, 1, T, E_, d_, h, d_, wr, d_, logits_.get(), E_, dt_, DType::Float32, s);
    hip::moe_route(logits_.as<float>(), T, E_, k_, coef_, idx_.as<int64_t>(), gsel_.as<float>(), probs_.as<float>(),
                   nullptr, counts_.as<int64_t>(), nullptr, aux, s);
    hip::moe_permute(idx_.as<int64_t>(), counts_.as<int64_t>(), T, k_, E_, offsets_.as<int64_t>(), dst_row_.as<int>(),
                     src_ent_.as<int>(), s);
    // expert row counts on the host: they size the per-expert GEMMs
    counts_h_.assign(E_, 0);
    offsets_h_.assign(E_ + 1, 0);
    AIC_HIP_CHECK(hipMemcpyAsync(counts_h_.data(), counts_.get(), sizeof(int64_t) * E_, hipMemcpyDeviceToHost, s));
    AIC_HIP_CHECK(hipMemcpyAsync(offsets_h_.data(), offsets_.get(), sizeof(int64_t) * (E_ + 1),
                                 hipMemcpyDeviceToHost, s));
    AIC_HIP_CHECK(hipStreamSynchronize(s));
    const int64_t used = offsets_h_[E_];
    xp_ = DeviceBuffer(es * used * d_, s);
    gu_ = DeviceBuffer(es * used * f2, s);
    a_ = DeviceBuffer(es * used * f_, s);
    ye_ = DeviceBuffer(es * used * d_, s);
    hip::moe_gather(h, d_, src_ent_.as<int>(), k_, used, d_, xp_.get(), dt_, s);
    auto at = [&](const DeviceBuffer& b, int64_t elem) { return static_cast<char*>(b.get()) + es * elem; };
    const char* exb = static_cast<const char*>(experts);
    // each expert's rows (a block of m rows starting at offsets_h_[e]) through its gate/up
    // projection, all experts in shared launches; then SwiGLU; then the down projections
    std::vector<hip::GemmArgs> v;
    for (int64_t e = 0; e < E_; ++e) {
        const int64_t m = offsets_h_[e + 1] - offsets_h_[e], o = offsets_h_[e];
        if (counts_h_[e] == 0) continue;
        v.push_back(args(0, 1, m, f2, d_, at(xp_, o * d_), d_, exb + es * e * ex, d_, at(gu_, o * f2), f2, dt_, dt_));
    }
    run_grouped(v, s);
    hip::swiglu_fwd(gu_.get(), at(gu_, f_), f2, a_.get(), f_, used, f_, dt_, s);
    v.clear();
    for (int64_t e = 0; e < E_; ++e) {
        const int64_t m = offsets_h_[e + 1] - offsets_h_[e], o = offsets_h_[e];
        if (counts_h_[e] == 0) continue;
        v.push_back(args(0, 1, m, d_, f_, at(a_, o * f_), f_, exb + es * (e * ex + 2 * f_ * d_), f_, at(ye_, o * d_),
                         d_, dt_, dt_));
    }
    run_grouped(v, s);
    hip::moe_combine(ye_.get(), idx_.as<int64_t>(), dst_row_.as<int>(), gsel_.as<float>(), T, k_, d_, R, d_, y, d_, dt_,
                     s);
}

void MoEFFN::backward(const void* dy, float daux, void* dh, float* dwr, float* dexperts, hipStream_t s,
                      const float* daux_scale) {
    AIC_CHECK(T_ > 0 && dy && dh && dwr && dexperts, InvalidArgument, "MoEFFN::backward: forward first, no nulls");
    const size_t es = dtype_size(dt_);
    const int64_t T = T_, f2 = 2 * f_, ex = 3 * f_ * d_, used = offsets_h_[E_];
    auto at = [&](const DeviceBuffer& b, int64_t elem) { return static_cast<char*>(b.get()) + es * elem; };
    DeviceBuffer dye(es * used * d_, s), dgsel(sizeof(float) * T * k_, s), da(es * used * f_, s),
        dgu(es * used * f2, s), dxp(es * used * d_, s), dlog(sizeof(float) * T * E_, s);
    hip::moe_combine_bwd(dy, d_, ye_.get(), src_ent_.as<int>(), gsel_.as<float>(), used, k_, d_, dye.get(),
                         dgsel.as<float>(), dt_, s);
    const char* exb = static_cast<const char*>(ex_);
    // down projections: da = dye . Wd and dWd = dye^T . a per expert, each kind in shared launches
    std::vector<hip::GemmArgs> vd, vw;
    for (int64_t e = 0; e < E_; ++e) {
        const int64_t m = offsets_h_[e + 1] - offsets_h_[e], o = offsets_h_[e];
        float* dgu_w = dexperts + e * ex;
        float* dd_w = dgu_w + 2 * f_ * d_;
        if (counts_h_[e] == 0) {
            AIC_HIP_CHECK(hipMemsetAsync(dgu_w, 0, sizeof(float) * ex, s));
            continue;
        }
        vd.push_back(args(0, 0, m, f_, d_, at(dye, o * d_), d_, exb + es * (e * ex + 2 * f_ * d_), f_, at(da, o * f_),
                          f_, dt_, dt_));
        vw.push_back(args(1, 0, d_, f_, m, at(dye, o * d_), d_, at(a_, o * f_), f_, dd_w, f_, dt_, DType::Float32));
    }
    run_grouped(vd, s);
    run_grouped(vw, s);
    hip::swiglu_bwd(gu_.get(), at(gu_, f_), f2, da.get(), f_, dgu.get(), at(dgu, f_), f2, used, f_, dt_, s);
    // gate/up projections: dxp = dgu . Wgu and dWgu = dgu^T . xp
    vd.clear();
    vw.clear();
    for (int64_t e = 0; e < E_; ++e) {
        const int64_t m = offsets_h_[e + 1] - offsets_h_[e], o = offsets_h_[e];
        if (counts_h_[e] == 0) continue;
        vd.push_back(args(0, 0, m, d_, f2, at(dgu, o * f2), f2, exb + es * e * ex, d_, at(dxp, o * d_), d_, dt_, dt_));
        vw.push_back(args(1, 0, f2, d_, m, at(dgu, o * f2), f2, at(xp_, o * d_), d_, dexperts + e * ex, d_, dt_,
                          DType::Float32));
    }
    run_grouped(vd, s);
    run_grouped(vw, s);
    hip::moe_scatter(dxp.get(), idx_.as<int64_t>(), dst_row_.as<int>(), T, k_, d_, dh, d_, false, dt_, s);
    // router: dlogits from the gates and the aux loss, then both router products
    hip::moe_router_bwd(probs_.as<float>(), idx_.as<int64_t>(), dgsel.as<float>(), counts_.as<int64_t>(), T, E_, k_,
                        coef_, daux, daux_scale, dlog.as<float>(), s);
    if (dt_ == DType::Float32) {
        gemm(1, 0, E_, d_, T, dlog.get(), E_, h_, d_, dwr, d_, DType::Float32, DType::Float32, s);
        gemm(0, 0, T, d_, E_, dlog.get(), E_, wr_, d_, dh, d_, DType::Float32, DType::Float32, s, 1.0f);
    } else {
        DeviceBuffer dlb(2 * T * E_, s);
        hip::cast_f32_bf16(dlog.as<float>(), dlb.get(), T * E_, s);
        gemm(1, 0, E_, d_, T, dlb.get(), E_, h_, d_, dwr, d_, DType::BFloat16, DType::Float32, s);
        gemm(0, 0, T, d_, E_, dlb.get(), E_, wr_, d_, dh, d_, DType::BFloat16, DType::BFloat16, s, 1.0f);
    }
}

}  // namespace aic::models
