// Shared device helpers for the gfx950 (CDNA4) kernels: bf16 conversion, vector types,
// wave64 reductions and launch checking.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../runtime/error.hpp"

namespace aic::hip {

using bf16 = __bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// float -> bf16, round to nearest even: the hardware conversion (v_cvt_pk_bf16_f32 on
// gfx950), equal to the reference's float_to_bf16 (include/core/dtype.hpp:118-126) for every
// non-NaN input; a NaN stays a NaN.
__device__ __forceinline__ bf16 f2bf(float f) { return static_cast<bf16>(f); }
__device__ __forceinline__ uint16_t f2bf_bits(float f) { return __builtin_bit_cast(uint16_t, f2bf(f)); }
// Two floats -> packed bf16 pair (low half = a), the same conversion as f2bf: one
// v_cvt_pk_bf16_f32 with both sources (converting the halves one at a time costs a shift and an
// or on top).
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const f32x2_v v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}
// The logistic sigmoid 1 / (1 + e^-x) with the hardware reciprocal (v_rcp_f32, within 1 ulp)
// instead of an IEEE division: the bf16 SwiGLU paths (GEMM epilogues and the standalone bf16
// passes, which must agree bit for bit) round the result to bf16 afterwards.
__device__ __forceinline__ float sigmoid_rcp(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float bf2f(bf16 h) {
    return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h)) << 16);
}

// Generic element load/store with fp32 compute.
template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i);
template <> __device__ __forceinline__ float ld<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float ld<bf16>(const bf16* p, int64_t i) { return bf2f(p[i]); }
template <typename T> __device__ __forceinline__ void st(T* p, int64_t i, float v);
template <> __device__ __forceinline__ void st<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void st<bf16>(bf16* p, int64_t i, float v) { p[i] = f2bf(v); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `red` is LDS of >= 16 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave, nw = blockDim.x / kWave;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float t = (threadIdx.x < nw) ? red[threadIdx.x] : 0.0f;
    if (w == 0) t = wave_sum(t);
    if (threadIdx.x == 0) red[0] = t;
    __syncthreads();
    return red[0];
}
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave, nw = blockDim.x / kWave;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float t = (threadIdx.x < nw) ? red[threadIdx.x] : -INFINITY;
    if (w == 0) t = wave_max(t);
    if (threadIdx.x == 0) red[0] = t;
    __syncthreads();
    return red[0];
}

// Direct global -> LDS copy of 16 (dma16) or 4 (dma4) bytes per lane: lane i's bytes land at
// lds + i * size (lds must be the same for the whole wave).  Issued as inline assembly so the
// compiler does not track it: the caller orders it with explicit s_waitcnt vmcnt(N) before the
// data is read (the compiler's own tracking would otherwise put a vmcnt(0) in front of every
// ds_read_b64_tr_b16, which carries no memory operand, and expose the whole copy latency).
__device__ __forceinline__ void dma16(const void* g, const void* lds) {
    const uint32_t l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(l)), "v"(g)
                 : "memory", "m0");
}
// The same with the global address as a wave-uniform base (SGPR pair) plus a per-lane 32-bit
// byte offset.
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, const void* lds) {
    const uint32_t l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    // readfirstlane returns int: each half goes through uint32_t so the low word is not
    // sign-extended into the high one
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
    const uint64_t bs = (static_cast<uint64_t>(hi) << 32) | lo;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(l)), "v"(voff), "s"(bs)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, const void* lds) {
    const uint32_t l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(l)), "v"(g)
                 : "memory", "m0");
}

inline unsigned grid_for(int64_t n, int block, int64_t cap = 65535LL * 8) {
    int64_t g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return static_cast<unsigned>(g);
}

}  // namespace aic::hip

#define AIC_LAUNCH_CHECK(what)                                                            \
    do {                                                                                  \
        hipError_t _e = hipGetLastError();                                                \
        AIC_CHECK(_e == hipSuccess, HipError, what, ": ", hipGetErrorString(_e));         \
    } while (0)
