// Per-kernel-class timing with HIP events on the stream the kernels run on.  When disabled,
// Scope objects cost one branch.  Events come from a pool that is reused after each
// collect().
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

namespace aic {

enum KernelClass : int {
    kGemmFwd = 0,  // y = x W^T      (transA 0, transB 1)
    kGemmDgrad,    // dx = dy W      (0, 0)
    kGemmWgrad,    // dW = dy^T x    (1, 0), fp32 output
    kAttnFwd,
    kAttnBwd,
    kNormFwd,
    kNormBwd,
    kRope,
    kSwigluFwd,
    kSwigluBwd,
    kCeFwd,
    kCeBwd,
    kCeFwdBwd,     // forward and backward in one pass (training steps)
    kEmbedFwd,
    kEmbedBwd,
    kGradNorm,
    kAdamW,
    kLora,         // LoRA adapter products (one pass over the large operand; HBM-bound)
    kNumKernelClasses
};

struct KernelClassStats {
    std::string name;
    long long launches = 0;
    double total_ms = 0.0;
    double flops = 0.0;
    double bytes = 0.0;
    bool mfma_bound = false;
};

class Profiler {
public:
    ~Profiler();
    void enable(bool on);
    // Classes timed while enabled: bit c for class c (all by default).  Recording an event pair
    // costs a few microseconds of queue time per launch, so a measurement that must not perturb
    // the step times only the class it reports.
    void set_mask(uint32_t mask) { mask_ = mask; }
    bool enabled() const { return on_; }
    static int class_index(const char* name);

    class Scope {
    public:
        Scope(Profiler* p, int cls, double flops, double bytes, hipStream_t s);
        ~Scope();
        Scope(const Scope&) = delete;
        Scope& operator=(const Scope&) = delete;

    private:
        Profiler* p_;
        hipStream_t s_;
        size_t idx_;
    };
    Scope scope(int cls, double flops, double bytes, hipStream_t s) { return Scope(this, cls, flops, bytes, s); }

    // Synchronises on the recorded events and folds them into the per-class totals.
    std::vector<KernelClassStats> collect();

private:
    struct Rec {
        int cls;
        double flops, bytes;
        hipEvent_t a, b;
    };
    hipEvent_t take();
    bool on_ = false;
    uint32_t mask_ = 0xffffffffu;
    std::vector<Rec> recs_;
    std::vector<hipEvent_t> pool_;
    size_t pool_used_ = 0;
    KernelClassStats totals_[kNumKernelClasses];
};

}  // namespace aic
