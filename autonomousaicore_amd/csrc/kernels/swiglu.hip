// SwiGLU activation h = silu(g) * u and its backward as single elementwise kernels over the
// fused gate/up projection output (the reference runs silu, mul and their backward nodes
// as separate ops, include/nn/swiglu.hpp:21-33, src/autograd/functions.cpp:60-68,167-175).
#include "common.hpp"
#include "kernels.hpp"

namespace aic::hip {

namespace {

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_k(const T* __restrict__ g, const T* __restrict__ u, int64_t ld_gu,
                                                    T* __restrict__ h, int64_t ld_h, int64_t T_rows, int f) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= T_rows * f) return;
    const int64_t t = idx / f;
    const int j = static_cast<int>(idx % f);
    const float x = ld(g, t * ld_gu + j);
    const float a = x / (1.0f + expf(-x));
    st(h, t * ld_h + j, a * ld(u, t * ld_gu + j));
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_k(const T* __restrict__ g, const T* __restrict__ u, int64_t ld_gu,
                                                    const T* __restrict__ dh, int64_t ld_h, T* dg, T* du,
                                                    int64_t ld_d, int64_t T_rows, int f) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= T_rows * f) return;
    const int64_t t = idx / f;
    const int j = static_cast<int>(idx % f);
    const float x = ld(g, t * ld_gu + j);
    const float uu = ld(u, t * ld_gu + j);
    const float d = ld(dh, t * ld_h + j);
    const float sg = sigmoidf_(x);
    const float a = x / (1.0f + expf(-x));
    const float ds = sg * (1.0f + x * (1.0f - sg));
    st(dg, t * ld_d + j, (d * uu) * ds);
    st(du, t * ld_d + j, d * a);
}

// bf16 fast path: 8 elements per thread with 16-byte accesses (f % 8 == 0, aligned).
__device__ __forceinline__ void unpack8(const uint4 v, float* o) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ uint4 pack8(const float* o) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = static_cast<uint32_t>(f2bf_bits(o[2 * i])) | (static_cast<uint32_t>(f2bf_bits(o[2 * i + 1])) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ __launch_bounds__(256) void swiglu_fwd_v8(const bf16* __restrict__ g, const bf16* __restrict__ u,
                                                     int64_t ld_gu, bf16* __restrict__ h, int64_t ld_h, int64_t T_rows,
                                                     int f) {
    const int per = f / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= T_rows * per) return;
    const int64_t t = idx / per;
    const int j = static_cast<int>(idx % per) * 8;
    float gv[8], uv[8], o[8];
    unpack8(*reinterpret_cast<const uint4*>(g + t * ld_gu + j), gv);
    unpack8(*reinterpret_cast<const uint4*>(u + t * ld_gu + j), uv);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (gv[i] * sigmoid_rcp(gv[i])) * uv[i];
    *reinterpret_cast<uint4*>(h + t * ld_h + j) = pack8(o);
}

__global__ __launch_bounds__(256) void swiglu_bwd_v8(const bf16* __restrict__ g, const bf16* __restrict__ u,
                                                     int64_t ld_gu, const bf16* __restrict__ dh, int64_t ld_h, bf16* dg,
                                                     bf16* du, int64_t ld_d, int64_t T_rows, int f) {
    const int per = f / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= T_rows * per) return;
    const int64_t t = idx / per;
    const int j = static_cast<int>(idx % per) * 8;
    float gv[8], uv[8], dv[8], og[8], ou[8];
    unpack8(*reinterpret_cast<const uint4*>(g + t * ld_gu + j), gv);
    unpack8(*reinterpret_cast<const uint4*>(u + t * ld_gu + j), uv);
    unpack8(*reinterpret_cast<const uint4*>(dh + t * ld_h + j), dv);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float sg = sigmoid_rcp(gv[i]);
        const float a = gv[i] * sg;
        og[i] = (dv[i] * uv[i]) * (sg * (1.0f + gv[i] * (1.0f - sg)));
        ou[i] = dv[i] * a;
    }
    *reinterpret_cast<uint4*>(dg + t * ld_d + j) = pack8(og);
    *reinterpret_cast<uint4*>(du + t * ld_d + j) = pack8(ou);
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

void swiglu_fwd(const void* g, const void* u, int64_t ld_gu, void* h, int64_t ld_h, int64_t T, int64_t f, DType dt,
                hipStream_t s) {
    AIC_CHECK(T >= 0 && f > 0 && ld_gu >= f && ld_h >= f, InvalidArgument, "swiglu_fwd: bad shape");
    if (T == 0) return;
    if (dt == DType::BFloat16 && f % 8 == 0 && ld_gu % 8 == 0 && ld_h % 8 == 0 && a16(g) && a16(u) && a16(h)) {
        const int64_t n = T * (f / 8);
        hipLaunchKernelGGL(swiglu_fwd_v8, dim3(grid_for(n, 256, 1LL << 31)), dim3(256), 0, s,
                           static_cast<const bf16*>(g), static_cast<const bf16*>(u), ld_gu, static_cast<bf16*>(h), ld_h,
                           T, static_cast<int>(f));
    } else if (dt == DType::BFloat16) {
        hipLaunchKernelGGL(swiglu_fwd_k<bf16>, dim3(grid_for(T * f, 256, 1LL << 31)), dim3(256), 0, s,
                           static_cast<const bf16*>(g), static_cast<const bf16*>(u), ld_gu, static_cast<bf16*>(h), ld_h,
                           T, static_cast<int>(f));
    } else if (dt == DType::Float32) {
        hipLaunchKernelGGL(swiglu_fwd_k<float>, dim3(grid_for(T * f, 256, 1LL << 31)), dim3(256), 0, s,
                           static_cast<const float*>(g), static_cast<const float*>(u), ld_gu, static_cast<float*>(h),
                           ld_h, T, static_cast<int>(f));
    } else {
        AIC_THROW(DTypeMismatch, "swiglu_fwd: dtype must be f32 or bf16");
    }
    AIC_LAUNCH_CHECK("swiglu_fwd");
}

void swiglu_bwd(const void* g, const void* u, int64_t ld_gu, const void* dh, int64_t ld_h, void* dg, void* du,
                int64_t ld_d, int64_t T, int64_t f, DType dt, hipStream_t s) {
    AIC_CHECK(T >= 0 && f > 0 && ld_gu >= f && ld_h >= f && ld_d >= f, InvalidArgument, "swiglu_bwd: bad shape");
    if (T == 0) return;
    if (dt == DType::BFloat16 && f % 8 == 0 && ld_gu % 8 == 0 && ld_h % 8 == 0 && ld_d % 8 == 0 && a16(g) && a16(u) &&
        a16(dh) && a16(dg) && a16(du)) {
        const int64_t n = T * (f / 8);
        hipLaunchKernelGGL(swiglu_bwd_v8, dim3(grid_for(n, 256, 1LL << 31)), dim3(256), 0, s,
                           static_cast<const bf16*>(g), static_cast<const bf16*>(u), ld_gu,
                           static_cast<const bf16*>(dh), ld_h, static_cast<bf16*>(dg), static_cast<bf16*>(du), ld_d, T,
                           static_cast<int>(f));
    } else if (dt == DType::BFloat16) {
        hipLaunchKernelGGL(swiglu_bwd_k<bf16>, dim3(grid_for(T * f, 256, 1LL << 31)), dim3(256), 0, s,
                           static_cast<const bf16*>(g), static_cast<const bf16*>(u), ld_gu,
                           static_cast<const bf16*>(dh), ld_h, static_cast<bf16*>(dg), static_cast<bf16*>(du), ld_d, T,
                           static_cast<int>(f));
    } else if (dt == DType::Float32) {
        hipLaunchKernelGGL(swiglu_bwd_k<float>, dim3(grid_for(T * f, 256, 1LL << 31)), dim3(256), 0, s,
                           static_cast<const float*>(g), static_cast<const float*>(u), ld_gu,
                           static_cast<const float*>(dh), ld_h, static_cast<float*>(dg), static_cast<float*>(du), ld_d,
                           T, static_cast<int>(f));
    } else {
        AIC_THROW(DTypeMismatch, "swiglu_bwd: dtype must be f32 or bf16");
    }
    AIC_LAUNCH_CHECK("swiglu_bwd");
}

}  // namespace aic::hip
