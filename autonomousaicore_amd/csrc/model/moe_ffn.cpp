#include "moe_ffn.hpp"

#include <algorithm>
#include <optional>
#include <vector>

#include "../kernels/gemm.hpp"
#include "../kernels/kernels.hpp"
#include "../runtime/error.hpp"

namespace aic::models {

namespace {

void gemm(int ta, int tb, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* B, int64_t ldb,
          void* C, int64_t ldc, DType ab, DType c, hipStream_t s, float beta = 0.0f, SqSlots sq = {}) {
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
    a.sq_part = sq.part;
    a.sq_nf = sq.nf;
    a.sq_cap = sq.cap;
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

// The experts' products of one kind in launches of up to 8 (hip::gemm_grouped); with sq, each
// launch's sums of squares go to its share of the region.
void run_grouped(std::vector<hip::GemmArgs> v, hipStream_t s, SqSlots sq = {}) {
    const size_t launches = (v.size() + 7) / 8;
    for (size_t i = 0; i < v.size(); i += 8) {
        if (sq.part) {
            const int64_t share = sq.cap / static_cast<int64_t>(launches), c = static_cast<int64_t>(i / 8);
            v[i].sq_part = sq.part + c * share;
            v[i].sq_nf = sq.nf + c * share;
            v[i].sq_cap = share;
        }
        hip::gemm_grouped(v.data() + i, static_cast<int>(std::min<size_t>(8, v.size() - i)), s);
    }
}

}  // namespace

MoEFFN::MoEFFN(int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, DType dt)
    : d_(d), f_(f), E_(E), k_(k), coef_(aux_coef), dt_(dt) {
    AIC_CHECK(d > 0 && f > 0 && E >= 1 && E <= 64 && k >= 1 && k <= 8 && k <= E, InvalidArgument,
              "MoEFFN: need d, f > 0, 1 <= E <= 64, 1 <= top_k <= min(E, 8)");
    AIC_CHECK(dt == DType::Float32 || dt == DType::BFloat16, DTypeMismatch, "MoEFFN: dtype must be f32 or bf16");
}

void MoEFFN::host_offsets(hipStream_t s) {
    if (host_valid_) return;
    counts_h_.assign(E_, 0);
    offsets_h_.assign(E_ + 1, 0);
    AIC_HIP_CHECK(hipMemcpyAsync(counts_h_.data(), counts_.get(), sizeof(int64_t) * E_, hipMemcpyDeviceToHost, s));
    AIC_HIP_CHECK(hipMemcpyAsync(offsets_h_.data(), offsets_.get(), sizeof(int64_t) * (E_ + 1),
                                 hipMemcpyDeviceToHost, s));
    AIC_HIP_CHECK(hipStreamSynchronize(s));
    host_valid_ = true;
}

const std::vector<int64_t>& MoEFFN::counts_host() {
    if (T_ == 0) {  // no forward yet: no routing
        counts_h_.clear();
        return counts_h_;
    }
    host_offsets(nullptr);
    return counts_h_;
}

// One kind of expert product: g is expert 0's product at row offset 0 (M or K: the rows).
// Ragged launch with the device offsets when the layout allows it, else one product per
// expert from the host offsets.
void MoEFFN::experts(const hip::GemmArgs& g, int ragged_k, int64_t b_stride, int64_t c_stride, hipStream_t s,
                     SqSlots sq, int cls, double flops) {
    std::optional<Profiler::Scope> scope;
    if (prof_ && cls >= 0) scope.emplace(prof_, cls, flops, 0.0, s);
    hip::RaggedArgs r;
    r.g = g;
    r.g.sq_part = sq.part;
    r.g.sq_nf = sq.nf;
    r.g.sq_cap = sq.cap;
    r.offsets = offsets_.as<int64_t>();
    r.E = static_cast<int>(E_);
    r.ragged_k = ragged_k;
    r.b_stride = b_stride;
    r.c_stride = c_stride;
    if (hip::gemm_ragged_eligible(r)) {
        hip::gemm_ragged(r, s);
        return;
    }
    host_offsets(s);
    const size_t es = dtype_size(dt_), ec = dtype_size(g.c);
    std::vector<hip::GemmArgs> v;
    for (int64_t e = 0; e < E_; ++e) {
        const int64_t m = offsets_h_[e + 1] - offsets_h_[e], o = offsets_h_[e];
        hip::GemmArgs a = g;
        if (ragged_k) {
            if (m == 0) {  // no rows: a zero gradient
                AIC_HIP_CHECK(hipMemsetAsync(static_cast<char*>(g.C) + ec * e * c_stride, 0,
                                             ec * static_cast<size_t>(g.M * g.ldc), s));
                continue;
            }
            a.K = m;
            a.A = static_cast<const char*>(g.A) + es * o * g.lda;
            a.B = static_cast<const char*>(g.B) + es * o * g.ldb;
            a.C = static_cast<char*>(g.C) + ec * e * c_stride;
        } else {
            if (m == 0) continue;
            a.M = m;
            a.A = static_cast<const char*>(g.A) + es * o * g.lda;
            a.B = static_cast<const char*>(g.B) + es * e * b_stride;
            a.C = static_cast<char*>(g.C) + ec * o * g.ldc;
        }
        a.sq_part = nullptr;
        a.glu_f = 0;
        a.glu_out = nullptr;
        a.dglu_gu = nullptr;
        a.dglu_out = nullptr;
        v.push_back(a);
    }
    run_grouped(std::move(v), s, sq);
    // SwiGLU of the products (the ragged launch does it in the epilogue)
    if (g.glu_f > 0)
        hip::swiglu_fwd(g.C, static_cast<const char*>(g.C) + es * g.glu_f, g.ldc, g.glu_out, g.ld_glu, g.M, g.glu_f,
                        g.c, s);
    if (g.dglu_gu)
        hip::swiglu_bwd(g.dglu_gu, static_cast<const char*>(g.dglu_gu) + es * g.N, g.dglu_ld, g.C, g.ldc, g.dglu_out,
                        static_cast<char*>(g.dglu_out) + es * g.N, g.dglu_ld, g.M, g.N, g.c, s);
}

void MoEFFN::forward(const void* h, int64_t T, const void* wr, const void* experts_w, const void* R, void* y,
                     float* aux, hipStream_t s) {
    AIC_CHECK(h && wr && experts_w && y && aux && T > 0, InvalidArgument, "MoEFFN::forward: bad arguments");
    const size_t es = dtype_size(dt_);
    const int64_t rows = hip::moe_max_rows(T, E_, k_), f2 = 2 * f_, ex = 3 * f_ * d_;
    T_ = T;
    h_ = h;
    wr_ = wr;
    ex_ = experts_w;
    logits_ = DeviceBuffer(sizeof(float) * T * E_, s);
    idx_ = DeviceBuffer(sizeof(int64_t) * T * k_, s);
    gsel_ = DeviceBuffer(sizeof(float) * T * k_, s);
    probs_ = DeviceBuffer(sizeof(float) * T * E_, s);
    counts_ = DeviceBuffer(sizeof(int64_t) * E_, s);
    offsets_ = DeviceBuffer(sizeof(int64_t) * (E_ + 1), s);
    dst_row_ = DeviceBuffer(sizeof(int) * T * k_, s);
    src_ent_ = DeviceBuffer(sizeof(int) * rows, s);
    host_valid_ = false;
    // router logits in fp32, routing, dispatch order
    gemm(0, 1, T, E_, d_, h, d_, wr, d_, logits_.get(), E_, dt_, DType::Float32, s);
    hip::moe_route(logits_.as<float>(), T, E_, k_, coef_, idx_.as<int64_t>(), gsel_.as<float>(), probs_.as<float>(),
                   nullptr, counts_.as<int64_t>(), nullptr, aux, s);
    hip::moe_permute(idx_.as<int64_t>(), counts_.as<int64_t>(), T, k_, E_, offsets_.as<int64_t>(), dst_row_.as<int>(),
                     src_ent_.as<int>(), s);
    // The expert products read the row offsets on the device (bf16), so the row passes and
    // buffers cover the bound `rows` (the rows after the experts' blocks are padding rows);
    // the fp32 path sizes everything from the host copy of the offsets.
    if (dt_ == DType::BFloat16) {
        used_ = rows;
    } else {
        host_offsets(s);
        used_ = offsets_h_[E_];
    }
    xp_ = DeviceBuffer(es * used_ * d_, s);
    gu_ = DeviceBuffer(es * used_ * f2, s);
    a_ = DeviceBuffer(es * used_ * f_, s);
    ye_ = DeviceBuffer(es * used_ * d_, s);
    hip::moe_gather(h, d_, src_ent_.as<int>(), k_, used_, d_, xp_.get(), dt_, s);
    const char* exb = static_cast<const char*>(experts_w);
    // gate/up of each expert's rows, SwiGLU, then the down projections
    hip::GemmArgs gu = args(0, 1, used_, f2, d_, xp_.get(), d_, exb, d_, gu_.get(), f2, dt_, dt_);
    gu.glu_f = f_;  // a = silu(gate) * up, in the product's epilogue where the shapes allow
    gu.glu_out = a_.get();
    gu.ld_glu = f_;
    const double routed = static_cast<double>(T) * k_, pf = 2.0 * routed * f_ * d_;  // FLOPs of an f x d product
    experts(gu, 0, ex, 0, s, {}, kGemmFwd, 2.0 * pf);
    experts(args(0, 1, used_, d_, f_, a_.get(), f_, exb + es * 2 * f_ * d_, f_, ye_.get(), d_, dt_, dt_), 0, ex, 0, s,
            {}, kGemmFwd, pf);
    hip::moe_combine(ye_.get(), idx_.as<int64_t>(), dst_row_.as<int>(), gsel_.as<float>(), T, k_, d_, R, d_, y, d_, dt_,
                     s);
}

void MoEFFN::backward(const void* dy, float daux, void* dh, float* dwr, float* dexperts, hipStream_t s,
                      const float* daux_scale, const SqSlots* sq) {
    const SqSlots sq_d = sq ? sq[0] : SqSlots{}, sq_gu = sq ? sq[1] : SqSlots{}, sq_r = sq ? sq[2] : SqSlots{};
    AIC_CHECK(T_ > 0 && dy && dh && dwr && dexperts, InvalidArgument, "MoEFFN::backward: forward first, no nulls");
    const size_t es = dtype_size(dt_);
    const int64_t T = T_, f2 = 2 * f_, ex = 3 * f_ * d_, used = used_;
    DeviceBuffer dye(es * used * d_, s), dgsel(sizeof(float) * T * k_, s), da(es * used * f_, s),
        dgu(es * used * f2, s), dxp(es * used * d_, s), dlog(sizeof(float) * T * E_, s);
    hip::moe_combine_bwd(dy, d_, ye_.get(), src_ent_.as<int>(), gsel_.as<float>(), used, k_, d_, dye.get(),
                         dgsel.as<float>(), dt_, s);
    const char* exb = static_cast<const char*>(ex_);
    // down projections: da = dye . Wd and dWd = dye^T . a (fp32, zero for an expert with no rows)
    // ... and da feeds SwiGLU's backward (dgu from da and the saved gate/up) in the product's
    // epilogue where the shapes allow
    hip::GemmArgs dn = args(0, 0, used, f_, d_, dye.get(), d_, exb + es * 2 * f_ * d_, f_, da.get(), f_, dt_, dt_);
    dn.dglu_gu = gu_.get();
    dn.dglu_out = dgu.get();
    dn.dglu_ld = f2;
    const double pf = 2.0 * static_cast<double>(T) * k_ * f_ * d_;  // FLOPs of an f x d product over the routed rows
    experts(dn, 0, ex, 0, s, {}, kGemmDgrad, pf);
    experts(args(1, 0, d_, f_, 0, dye.get(), d_, a_.get(), f_, dexperts + 2 * f_ * d_, f_, dt_, DType::Float32), 1, 0,
            ex, s, sq_d, kGemmWgrad, pf);
    // gate/up projections: dxp = dgu . Wgu and dWgu = dgu^T . xp
    experts(args(0, 0, used, d_, f2, dgu.get(), f2, exb, d_, dxp.get(), d_, dt_, dt_), 0, ex, 0, s, {}, kGemmDgrad,
            2.0 * pf);
    experts(args(1, 0, f2, d_, 0, dgu.get(), f2, xp_.get(), d_, dexperts, d_, dt_, DType::Float32), 1, 0, ex, s, sq_gu,
            kGemmWgrad, 2.0 * pf);
    // router: dlogits from the gates and the aux loss, then both router products (for bf16 the
    // input gradient dlogits . W_r joins the experts' sum in the scatter, in fp32)
    hip::moe_router_bwd(probs_.as<float>(), idx_.as<int64_t>(), dgsel.as<float>(), counts_.as<int64_t>(), T, E_, k_,
                        coef_, daux, daux_scale, dlog.as<float>(), s);
    if (dt_ == DType::Float32) {
        hip::moe_scatter(dxp.get(), idx_.as<int64_t>(), dst_row_.as<int>(), T, k_, d_, dh, d_, false, dt_, s);
        gemm(1, 0, E_, d_, T, dlog.get(), E_, h_, d_, dwr, d_, DType::Float32, DType::Float32, s, 0.0f, sq_r);
        gemm(0, 0, T, d_, E_, dlog.get(), E_, wr_, d_, dh, d_, DType::Float32, DType::Float32, s, 1.0f);
    } else {
        hip::moe_scatter(dxp.get(), idx_.as<int64_t>(), dst_row_.as<int>(), T, k_, d_, dh, d_, false, dt_, s,
                         dlog.as<float>(), wr_, E_);
        DeviceBuffer dlb(2 * T * E_, s);
        hip::cast_f32_bf16(dlog.as<float>(), dlb.get(), T * E_, s);
        gemm(1, 0, E_, d_, T, dlb.get(), E_, h_, d_, dwr, d_, DType::BFloat16, DType::Float32, s, 0.0f, sq_r);
    }
}

}  // namespace aic::models
