// Streaming probe: the HBM rate that a single pass in the library's own streaming form reaches
// for a given mix of fp32 reads and writes on this GPU.  The form is adamw_k's: 256 threads,
// two float4 groups per thread per iteration (all of a group's loads issued before any use),
// a grid-stride loop, plain or non-temporal accesses.  It has no counterpart in the reference;
// it is the measured ceiling against which the bandwidth-bound kernels (AdamW: 4 reads, 3 fp32
// writes and a bf16 copy per element) are judged, beside torch's own device copy and add.
#include "../../../include/aic_hip.h"
#include "common.hpp"
#include "kernels.hpp"

namespace aic::hip {

namespace {

struct ProbeArgs {
    const float* in[4];
    float* out[3];
    bf16* out_bf16;
    float* sink;
};

template <bool NT>
__device__ __forceinline__ f32x4 ld4(const float* p, int64_t i) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + i);
    else return reinterpret_cast<const f32x4*>(p)[i];
}

template <bool NT, typename V>
__device__ __forceinline__ void st(V* p, int64_t i, V v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p + i);
    else p[i] = v;
}

// out_j = (sum of the inputs) + j; out_bf16 = bf16(sum); with no output at all, a thread whose
// sums are all zero writes 0 to sink[0] (so the loads stay live; every such write stores 0).
template <int NI, int NO, bool B16, bool NT>
__global__ __launch_bounds__(256) void stream_probe_k(const ProbeArgs a, int64_t n4) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * blockDim.x * 2 + threadIdx.x; base < n4; base += 2 * stride) {
        f32x4 x[2][NI > 0 ? NI : 1];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t i = base + u * blockDim.x;
            if (i < n4) {
#pragma unroll
                for (int k = 0; k < NI; ++k) x[u][k] = ld4<NT>(a.in[k], i);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t i = base + u * blockDim.x;
            if (i >= n4) continue;
            f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < NI; ++k) s += x[u][k];
#pragma unroll
            for (int j = 0; j < NO; ++j) st<NT>(reinterpret_cast<f32x4*>(a.out[j]), i, s + static_cast<float>(j));
            if constexpr (B16) {
                u32x2 w;
                w[0] = static_cast<uint32_t>(f2bf_bits(s[0])) | (static_cast<uint32_t>(f2bf_bits(s[1])) << 16);
                w[1] = static_cast<uint32_t>(f2bf_bits(s[2])) | (static_cast<uint32_t>(f2bf_bits(s[3])) << 16);
                st<NT>(reinterpret_cast<u32x2*>(a.out_bf16), i, w);
            }
            if constexpr (NO == 0 && !B16) {
                if (s[0] == 0.0f && s[1] == 0.0f && s[2] == 0.0f && s[3] == 0.0f) a.sink[0] = 0.0f;
            }
        }
    }
}

template <int NI, int NO, bool B16>
void launch(const ProbeArgs& a, int64_t n, bool nt, hipStream_t s) {
    const unsigned grid = grid_for((n + 7) / 8, 256, 262144);  // as adamw_multi sizes its grid
    if (nt) hipLaunchKernelGGL((stream_probe_k<NI, NO, B16, true>), dim3(grid), dim3(256), 0, s, a, n / 4);
    else hipLaunchKernelGGL((stream_probe_k<NI, NO, B16, false>), dim3(grid), dim3(256), 0, s, a, n / 4);
    AIC_LAUNCH_CHECK("stream_probe");
}

}  // namespace

void stream_probe(const float* const* in, int n_in, float* const* out, int n_out, void* out_bf16, float* sink,
                  int64_t n, bool nontemporal, hipStream_t s) {
    AIC_CHECK(n >= 0 && n % 4 == 0, InvalidArgument, "stream_probe: n must be a non-negative multiple of 4");
    AIC_CHECK(n_in >= 0 && n_in <= 4 && n_out >= 0 && n_out <= 3, InvalidArgument,
              "stream_probe: at most 4 inputs and 3 outputs");
    ProbeArgs a{};
    uintptr_t bits = 0;
    for (int k = 0; k < n_in; ++k) {
        AIC_CHECK(in && in[k], InvalidArgument, "stream_probe: null input");
        a.in[k] = in[k];
        bits |= reinterpret_cast<uintptr_t>(in[k]);
    }
    for (int j = 0; j < n_out; ++j) {
        AIC_CHECK(out && out[j], InvalidArgument, "stream_probe: null output");
        a.out[j] = out[j];
        bits |= reinterpret_cast<uintptr_t>(out[j]);
    }
    a.out_bf16 = static_cast<bf16*>(out_bf16);
    a.sink = sink;
    AIC_CHECK((bits & 15u) == 0 && (reinterpret_cast<uintptr_t>(out_bf16) & 7u) == 0, InvalidArgument,
              "stream_probe: fp32 buffers must be 16-byte and the bf16 buffer 8-byte aligned");
    const bool b16 = out_bf16 != nullptr;
    AIC_CHECK(n_out > 0 || b16 || sink, InvalidArgument, "stream_probe: a read-only pass needs sink");
    if (n == 0) return;
    // the mixes the bandwidth-bound kernels use: read, write, copy, add (2 reads + 1 write),
    // and AdamW's 4 reads + 3 writes + bf16 copy
    if (n_in == 1 && n_out == 0 && !b16) launch<1, 0, false>(a, n, nontemporal, s);
    else if (n_in == 0 && n_out == 1 && !b16) launch<0, 1, false>(a, n, nontemporal, s);
    else if (n_in == 1 && n_out == 1 && !b16) launch<1, 1, false>(a, n, nontemporal, s);
    else if (n_in == 2 && n_out == 1 && !b16) launch<2, 1, false>(a, n, nontemporal, s);
    else if (n_in == 4 && n_out == 3 && b16) launch<4, 3, true>(a, n, nontemporal, s);
    else AIC_CHECK(false, InvalidArgument, "stream_probe: mix not provided (read, write, copy, add, AdamW)");
}

}  // namespace aic::hip
