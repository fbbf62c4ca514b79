// INT4 symmetric weight quantization for the QLoRA base weights.
//
// Replaces QuantizedTensor::quantize / dequantize for INT4_SYMMETRIC (src/nn/quantization.cpp:
// 197-295 and 359-474) and the CUDA launcher launch_dequantize_int4 (src/cuda/cuda_quantize.cu:
// 54-94, 141-159).  The reference quantizes on the host and dequantizes to a fresh fp32 tensor
// on every QuantizedLinear::forward; here both run on the device and the dequantized weight is
// written straight in the GEMM's operand type (bf16 for AMP), so one pass reads 0.5 B and writes
// 2 B per weight.
//
// Format (shared with the reference, bit for bit):
//   groups of G consecutive elements of the flat row-major weight (G <= 0 or G > n: one group);
//   s = max(absmax / 7, 1e-8); q = clamp(round_half_away(x / s), -7, 7);
//   byte i holds element 2i in its low nibble and element 2i+1 in its high nibble, as 4-bit two's
//   complement (include/nn/quantization.hpp:41-56); deq = q * s.
// Scales are stored as fp32 (the reference) or fp16 (the QLoRA configuration); q always uses the
// fp32 s, so the packed bytes are the reference's either way.  An odd G with more than one group
// is rejected: the reference would then write two groups into one byte.
#include "common.hpp"
#include "kernels.hpp"

namespace aic::hip {

namespace {

__device__ __forceinline__ float scale_at(const void* scales, bool f16, int64_t g) {
    return f16 ? static_cast<float>(static_cast<const _Float16*>(scales)[g]) : static_cast<const float*>(scales)[g];
}

__device__ __forceinline__ unsigned quant_nibble(float x, float s) {
    float q = roundf(x / s);  // correctly rounded division, then halves away from zero (std::round)
    q = fminf(fmaxf(q, -7.0f), 7.0f);
    return static_cast<unsigned>(static_cast<int>(q)) & 0x0fu;
}

__device__ __forceinline__ float nibble_val(unsigned u) { return static_cast<float>(static_cast<int>(u << 28) >> 28); }

// One 256-thread block per group: absmax (exact in any order), the scale, then one byte per
// element pair.  Groups start on even elements, so every byte belongs to one group.
__global__ __launch_bounds__(256) void int4_quantize_k(const float* __restrict__ x, int64_t n, int64_t G,
                                                       uint8_t* __restrict__ packed, void* __restrict__ scales,
                                                       bool f16) {
    __shared__ float red[16];
    const int64_t g = blockIdx.x, start = g * G, end = start + G < n ? start + G : n;
    float amax = 0.0f;
    for (int64_t i = start + threadIdx.x; i < end; i += blockDim.x) amax = fmaxf(amax, fabsf(x[i]));
    amax = block_max(amax, red);
    float s = amax / 7.0f;
    if (s < 1e-8f) s = 1e-8f;
    if (threadIdx.x == 0) {
        if (f16) static_cast<_Float16*>(scales)[g] = static_cast<_Float16>(s);
        else static_cast<float*>(scales)[g] = s;
    }
    for (int64_t i = start + 2 * static_cast<int64_t>(threadIdx.x); i < end; i += 2 * blockDim.x) {
        const unsigned lo = quant_nibble(x[i], s);
        const unsigned hi = i + 1 < end ? quant_nibble(x[i + 1], s) : 0u;
        packed[i / 2] = static_cast<uint8_t>(lo | (hi << 4));
    }
}

template <typename OT> struct Out8;
template <> struct Out8<float> {
    static __device__ __forceinline__ void store(float* o, const float (&v)[8]) {
        reinterpret_cast<float4*>(o)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(o)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
};
template <> struct Out8<bf16> {
    static __device__ __forceinline__ void store(bf16* o, const float (&v)[8]) {
        *reinterpret_cast<uint4*>(o) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                  pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
    }
};

// Eight elements (four packed bytes) per thread.  G8: G is a multiple of 8, so the eight share
// one scale and the loads and stores are full vectors; otherwise per-element scales.
template <typename OT, bool G8>
__global__ __launch_bounds__(256) void int4_dequant_k(const uint8_t* __restrict__ packed, const void* __restrict__ scales,
                                                      bool f16, int64_t n, int64_t G, OT* __restrict__ out) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x, i0 = 8 * c;
    if (i0 >= n) return;
    if (G8 && i0 + 8 <= n) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(packed + 4 * c);
        const float s = scale_at(scales, f16, i0 / G);
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = nibble_val((w >> (4 * j)) & 0x0fu) * s;
        Out8<OT>::store(out + i0, v);
        return;
    }
    const int64_t e = i0 + 8 < n ? i0 + 8 : n;
    for (int64_t i = i0; i < e; ++i) {
        const unsigned b = packed[i / 2], u = (i & 1) ? (b >> 4) : (b & 0x0fu);
        st<OT>(out, i, nibble_val(u) * scale_at(scales, f16, i / G));
    }
}

// The CUDA launcher's general form (zero points, signed or unsigned nibbles; fp32 scales and
// output): element i = (val - zp[i / G]) * s[i / G], G <= 0 meaning one group, any G (each
// element finds its own group); eight elements (four bytes) per thread.
__global__ __launch_bounds__(256) void int4_dequant_zp_k(const uint8_t* __restrict__ packed,
                                                         const float* __restrict__ scales,
                                                         const float* __restrict__ zp, bool is_signed, int64_t n,
                                                         int64_t G, float* __restrict__ out) {
    const int64_t i0 = 8 * (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x);
    if (i0 >= n) return;
    const int64_t e = i0 + 8 < n ? i0 + 8 : n;
    for (int64_t i = i0; i < e; ++i) {
        const unsigned b = packed[i / 2], u = (i & 1) ? (b >> 4) : (b & 0x0fu);
        const float val = is_signed ? nibble_val(u) : static_cast<float>(u);
        const int64_t g = G > 0 ? i / G : 0;
        out[i] = (val - (zp ? zp[g] : 0.0f)) * scales[g];
    }
}

}  // namespace

void int4_dequant_zp(const uint8_t* packed, const float* scales, const float* zp, bool is_signed, int64_t n,
                     int64_t G, float* out, hipStream_t s) {
    AIC_CHECK(n >= 0, InvalidArgument, "int4_dequant_zp: negative element count");
    if (n == 0) return;
    AIC_CHECK(packed && scales && out, InvalidArgument, "int4_dequant_zp: null pointer");
    const int64_t blocks = ((n + 7) / 8 + 255) / 256;
    AIC_CHECK(blocks < (1LL << 31), InvalidArgument, "int4_dequant_zp: too many elements");
    hipLaunchKernelGGL(int4_dequant_zp_k, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, packed, scales, zp,
                       is_signed, n, G, out);
    AIC_LAUNCH_CHECK("int4_dequant_zp");
}

int64_t int4_group(int64_t n, int64_t G) {
    AIC_CHECK(n >= 0, InvalidArgument, "int4: negative element count");
    if (G <= 0 || G > n) G = n > 0 ? n : 1;
    AIC_CHECK((n + G - 1) / G <= 1 || G % 2 == 0, InvalidArgument,
              "int4: the group size must be even when there is more than one group (got ", G, ")");
    return G;
}

void int4_quantize(const float* x, int64_t n, int64_t G, uint8_t* packed, void* scales, DType scale_t, hipStream_t s) {
    G = int4_group(n, G);
    AIC_CHECK(scale_t == DType::Float32 || scale_t == DType::Float16, DTypeMismatch, "int4: scales must be f32 or f16");
    if (n == 0) return;
    AIC_CHECK(x && packed && scales, InvalidArgument, "int4_quantize: null pointer");
    const int64_t ng = (n + G - 1) / G;
    AIC_CHECK(ng < (1LL << 31), InvalidArgument, "int4_quantize: too many groups");
    hipLaunchKernelGGL(int4_quantize_k, dim3(static_cast<unsigned>(ng)), dim3(256), 0, s, x, n, G, packed, scales,
                       scale_t == DType::Float16);
    AIC_LAUNCH_CHECK("int4_quantize");
}

void int4_dequant(const uint8_t* packed, const void* scales, DType scale_t, int64_t n, int64_t G, void* out, DType out_t,
                  hipStream_t s) {
    G = int4_group(n, G);
    AIC_CHECK(scale_t == DType::Float32 || scale_t == DType::Float16, DTypeMismatch, "int4: scales must be f32 or f16");
    AIC_CHECK(out_t == DType::Float32 || out_t == DType::BFloat16, DTypeMismatch, "int4_dequant: output must be f32 or bf16");
    if (n == 0) return;
    AIC_CHECK(packed && scales && out, InvalidArgument, "int4_dequant: null pointer");
    const bool g8 = G % 8 == 0 && reinterpret_cast<uintptr_t>(packed) % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const int64_t chunks = (n + 7) / 8, blocks = (chunks + 255) / 256;
    AIC_CHECK(blocks < (1LL << 31), InvalidArgument, "int4_dequant: too many elements");
    const bool f16 = scale_t == DType::Float16;
    const dim3 grid(static_cast<unsigned>(blocks)), block(256);
    if (out_t == DType::Float32) {
        if (g8) hipLaunchKernelGGL((int4_dequant_k<float, true>), grid, block, 0, s, packed, scales, f16, n, G, static_cast<float*>(out));
        else hipLaunchKernelGGL((int4_dequant_k<float, false>), grid, block, 0, s, packed, scales, f16, n, G, static_cast<float*>(out));
    } else {
        if (g8) hipLaunchKernelGGL((int4_dequant_k<bf16, true>), grid, block, 0, s, packed, scales, f16, n, G, static_cast<bf16*>(out));
        else hipLaunchKernelGGL((int4_dequant_k<bf16, false>), grid, block, 0, s, packed, scales, f16, n, G, static_cast<bf16*>(out));
    }
    AIC_LAUNCH_CHECK("int4_dequant");
}

}  // namespace aic::hip
