#include "profiler.hpp"

#include <cstring>

#include "error.hpp"

namespace aic {

namespace {
const char* kNames[kNumKernelClasses] = {"gemm_fwd",   "gemm_dgrad", "gemm_wgrad", "attn_fwd",   "attn_bwd",
                                          "rmsnorm_fwd", "rmsnorm_bwd", "rope",      "swiglu_fwd", "swiglu_bwd",
                                          "ce_fwd",     "ce_bwd",     "ce_fwd_bwd", "embed_fwd",  "embed_bwd",
                                          "grad_norm",  "adamw",      "lora"};
const bool kMfma[kNumKernelClasses] = {true,  true,  true,  true,  true,  false, false, false, false,
                                       false, false, false, false, false, false, false, false, false};
}  // namespace

int Profiler::class_index(const char* name) {
    for (int c = 0; c < kNumKernelClasses; ++c)
        if (name && std::strcmp(name, kNames[c]) == 0) return c;
    return -1;
}

Profiler::~Profiler() {
    for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
}

void Profiler::enable(bool on) {
    on_ = on;
    if (on) {
        recs_.clear();
        pool_used_ = 0;
        for (int c = 0; c < kNumKernelClasses; ++c) {
            totals_[c] = KernelClassStats{};
            totals_[c].name = kNames[c];
            totals_[c].mfma_bound = kMfma[c];
        }
    }
}

hipEvent_t Profiler::take() {
    if (pool_used_ == pool_.size()) {
        hipEvent_t e;
        AIC_HIP_CHECK(hipEventCreate(&e));
        pool_.push_back(e);
    }
    return pool_[pool_used_++];
}

Profiler::Scope::Scope(Profiler* p, int cls, double flops, double bytes, hipStream_t s)
    : p_(p->on_ && ((p->mask_ >> cls) & 1u) ? p : nullptr), s_(s), idx_(0) {
    if (!p_) return;
    Rec r{cls, flops, bytes, p_->take(), p_->take()};
    AIC_HIP_CHECK(hipEventRecord(r.a, s));
    idx_ = p_->recs_.size();
    p_->recs_.push_back(r);
}

Profiler::Scope::~Scope() {
    if (p_) (void)hipEventRecord(p_->recs_[idx_].b, s_);
}

std::vector<KernelClassStats> Profiler::collect() {
    for (const Rec& r : recs_) {
        AIC_HIP_CHECK(hipEventSynchronize(r.b));
        float ms = 0.0f;
        AIC_HIP_CHECK(hipEventElapsedTime(&ms, r.a, r.b));
        KernelClassStats& t = totals_[r.cls];
        t.launches += 1;
        t.total_ms += ms;
        t.flops += r.flops;
        t.bytes += r.bytes;
    }
    recs_.clear();
    pool_used_ = 0;
    std::vector<KernelClassStats> out;
    for (int c = 0; c < kNumKernelClasses; ++c)
        if (totals_[c].launches > 0) out.push_back(totals_[c]);
    return out;
}

}  // namespace aic
