// Mixture-of-experts feed-forward block of MoETransformerBlock (src/nn/moe.cpp:155-253):
// router Linear(d, E) -> top-k routing with normalised gates and the load-balancing aux loss,
// E SwiGLU experts (gate [f,d], up [f,d], down [d,f], no bias) on the tokens routed to them,
// gate-weighted combine; and the backward of all of it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "../kernels/gemm.hpp"
#include "../runtime/dtype.hpp"
#include "../runtime/memory_pool.hpp"
#include "../runtime/profiler.hpp"

namespace aic::models {

// A slot region for the sums of squares of an fp32 weight gradient (GemmArgs::sq_*).
struct SqSlots {
    double* part = nullptr;
    int* nf = nullptr;
    int64_t cap = 0;
};

class MoEFFN {
public:
    MoEFFN(int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, DType dt);

    // h [T, d] (dt, leading dimension d); router wr [E, d] (dt); experts: E consecutive blocks of
    // gate [f, d], up [f, d], down [d, f] (dt).  y [T, d] (dt) = R + MoE(h) (R nullable);
    // *aux (device fp32) = the aux loss.  The inputs stay referenced until backward.
    void forward(const void* h, int64_t T, const void* wr, const void* experts, const void* R, void* y, float* aux,
                 hipStream_t s);
    // dy [T, d] (dt), daux = dL/daux.  dh [T, d] (dt) is overwritten; dwr [E, d] and dexperts (the
    // experts layout, fp32) are overwritten (zero for an expert that received no token).
    // daux_scale (device, nullable) multiplies daux (the loss scale of an AMP step).  sq (nullable):
    // slot regions for the sums of squares of the down, gate/up and router weight gradients.
    void backward(const void* dy, float daux, void* dh, float* dwr, float* dexperts, hipStream_t s,
                  const float* daux_scale = nullptr, const SqSlots* sq = nullptr);

    // Routing of the last forward: idx [T, k] and counts [E] (device pointers).
    const int64_t* idx() const { return idx_.as<int64_t>(); }
    const int64_t* counts() const { return counts_.as<int64_t>(); }
    int64_t tokens() const { return T_; }
    int64_t top_k() const { return k_; }
    // counts on the host (copied from the device, with a stream synchronisation, on first use)
    const std::vector<int64_t>& counts_host();
    // Times the experts' products under the GEMM classes of `p` (nullable), with the FLOPs of the
    // routed rows (T top_k; the padding rows of the device-offset launches are not counted).
    void set_profiler(Profiler* p) { prof_ = p; }

private:
    int64_t d_, f_, E_, k_;
    float coef_;
    DType dt_;
    int64_t T_ = 0;
    const void* h_ = nullptr;
    const void* wr_ = nullptr;
    const void* ex_ = nullptr;
    void host_offsets(hipStream_t s);
    void experts(const hip::GemmArgs& g, int ragged_k, int64_t b_stride, int64_t c_stride, hipStream_t s,
                 SqSlots sq = {}, int cls = -1, double flops = 0.0);
    Profiler* prof_ = nullptr;
    int64_t used_ = 0;  // rows of the permuted buffers
    bool host_valid_ = false;
    std::vector<int64_t> counts_h_, offsets_h_;
    DeviceBuffer logits_, idx_, gsel_, probs_, counts_, offsets_, dst_row_, src_ent_, xp_, gu_, a_, ye_;
};

}  // namespace aic::models
