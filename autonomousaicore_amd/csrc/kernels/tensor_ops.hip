// Tensor primitives of the reference's backend: strided copy (contiguous / clone), dtype casts,
// broadcasting elementwise binary ops, unary functions, full and per-dimension reductions, cat
// and the broadcast-gradient reduction of autograd.
//
// Replaces (paths relative to the reference repository's AutonomousAICore/):
//   Tensor::clone / contiguous for a strided view (src/tensor/tensor.cpp:248-304), whose GPU
//     path copies to the host, walks the multi-index there and copies back;
//   Tensor::to(DType) (src/tensor/tensor.cpp:359-410), also a host round trip on the GPU;
//   aic::cuda::add/sub/mul/div/neg/abs/exp/log/sqrt/tanh/sigmoid/gelu/silu
//     (src/cuda/cuda_elementwise.cuh:9-22; CPU semantics src/ops/cpu_ops.cpp:14-146);
//   aic::cuda::sum/mean/max/min, full and along a dim (src/cuda/cuda_reductions.cuh:10-18; CPU
//     semantics src/ops/cpu_ops.cpp:151-287), which run one thread per output;
//   cat (src/ops/ops.cpp:473-530) and reduce_gradient_for_broadcast
//     (src/autograd/functions.cpp:10-41).
// All of it is HBM-bound: vectorised loads where the layout allows, one pass per op.
// Semantics kept from the reference CPU path: fp32 compute; sums accumulate in double (the GPU
// sums in double too, in a fixed tree order, so results are deterministic and equal to the
// sequential double sum up to double rounding); max / min never take a NaN; a full mean is
// float(sum) / float(n), a per-dim mean float(sum / n) in double; float -> f16 / bf16 and
// f16 -> float follow include/core/dtype.hpp:65-133 bit for bit (round to nearest even, the
// reference's NaN encodings).
#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

constexpr int kMaxDims = 8;

struct View {
    int64_t shape[kMaxDims];
    int64_t strides[kMaxDims];
    int64_t offset;
    int ndim;
};

// ---------------------------------------------------------------- strided copy
template <typename T>
__global__ __launch_bounds__(256) void strided_copy_k(const T* __restrict__ src, View v, T* __restrict__ dst,
                                                      int64_t total) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t rem = i, off = v.offset;
        for (int d = v.ndim - 1; d >= 0; --d) {
            const int64_t c = rem % v.shape[d];
            rem /= v.shape[d];
            off += c * v.strides[d];
        }
        dst[i] = src[off];
    }
}

// ---------------------------------------------------------------- casts
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    const uint32_t x = __float_as_uint(f), sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x007FFFFFu;
    const int32_t exp = static_cast<int32_t>((x >> 23) & 0xFFu);
    if (exp == 0xFF) return static_cast<uint16_t>(sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    const int32_t e = exp - 127 + 15;
    if (e >= 0x1F) return static_cast<uint16_t>(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        mant |= 0x00800000u;
        const uint32_t shift = static_cast<uint32_t>(14 - e);
        uint32_t hm = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (hm & 1u))) ++hm;
        return static_cast<uint16_t>(sign | hm);
    }
    uint32_t h = sign | (static_cast<uint32_t>(e) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return static_cast<uint16_t>(h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu;
    const uint32_t mant = h & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return __uint_as_float(sign);
        const int lz = __clz(mant) - 21;  // shifts that bring the leading one to bit 10
        return __uint_as_float(sign | (static_cast<uint32_t>(113 - lz) << 23) | (((mant << lz) & 0x3FFu) << 13));
    }
    if (exp == 0x1F) return __uint_as_float(sign | 0x7F800000u | (mant << 13));
    return __uint_as_float(sign | ((exp + 112u) << 23) | (mant << 13));
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    const uint32_t x = __float_as_uint(f);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x007FFFFFu) != 0)
        return static_cast<uint16_t>(((x >> 16) & 0x8000u) | 0x7FC0u);
    return static_cast<uint16_t>((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

// codes as aic::DType: 0 f32, 1 f16, 2 bf16, 3 i32, 4 i64
template <int FROM, int TO>
__global__ __launch_bounds__(256) void cast_k(const void* __restrict__ src, void* __restrict__ dst, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if constexpr (FROM == 0 && TO == 1)
            static_cast<uint16_t*>(dst)[i] = f32_to_f16_bits(static_cast<const float*>(src)[i]);
        else if constexpr (FROM == 0 && TO == 2)
            static_cast<uint16_t*>(dst)[i] = f32_to_bf16_bits(static_cast<const float*>(src)[i]);
        else if constexpr (FROM == 1 && TO == 0)
            static_cast<float*>(dst)[i] = f16_bits_to_f32(static_cast<const uint16_t*>(src)[i]);
        else if constexpr (FROM == 2 && TO == 0)
            static_cast<float*>(dst)[i] = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(src)[i]) << 16);
        else if constexpr (FROM == 0 && TO == 4)
            static_cast<int64_t*>(dst)[i] = static_cast<int64_t>(static_cast<const float*>(src)[i]);
        else if constexpr (FROM == 4 && TO == 0)
            static_cast<float*>(dst)[i] = static_cast<float>(static_cast<const int64_t*>(src)[i]);
        else if constexpr (FROM == 0 && TO == 3)
            static_cast<int32_t*>(dst)[i] = static_cast<int32_t>(static_cast<const float*>(src)[i]);
        else if constexpr (FROM == 3 && TO == 0)
            static_cast<float*>(dst)[i] = static_cast<float>(static_cast<const int32_t*>(src)[i]);
        else if constexpr (FROM == 4 && TO == 3)
            static_cast<int32_t*>(dst)[i] = static_cast<int32_t>(static_cast<const int64_t*>(src)[i]);
        else
            static_cast<int64_t*>(dst)[i] = static_cast<int64_t>(static_cast<const int32_t*>(src)[i]);
    }
}

// ---------------------------------------------------------------- binary / unary
__device__ __forceinline__ float bin(int op, float x, float y) {
    switch (op) {
        case 0: return x + y;
        case 1: return x - y;
        case 2: return x * y;
        default: return x / y;
    }
}

// Same shape, both contiguous: four elements per thread.
__global__ __launch_bounds__(256) void binary_flat_k(int op, const float* __restrict__ a, const float* __restrict__ b,
                                                     float* __restrict__ out, int64_t n) {
    const int64_t n4 = n / 4;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const float4 x = reinterpret_cast<const float4*>(a)[i], y = reinterpret_cast<const float4*>(b)[i];
        reinterpret_cast<float4*>(out)[i] = make_float4(bin(op, x.x, y.x), bin(op, x.y, y.y), bin(op, x.z, y.z),
                                                        bin(op, x.w, y.w));
    }
    for (int64_t i = 4 * n4 + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[i] = bin(op, a[i], b[i]);
}

// General case: the output's multi-index mapped through both operands' broadcast strides.
__global__ __launch_bounds__(256) void binary_bcast_k(int op, const float* __restrict__ a, View va,
                                                      const float* __restrict__ b, View vb, float* __restrict__ out,
                                                      int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t rem = i, oa = va.offset, ob = vb.offset;
        for (int d = va.ndim - 1; d >= 0; --d) {
            const int64_t c = rem % va.shape[d];
            rem /= va.shape[d];
            oa += c * va.strides[d];
            ob += c * vb.strides[d];
        }
        out[i] = bin(op, a[oa], b[ob]);
    }
}

__device__ __forceinline__ float una(int op, float v) {
    switch (op) {
        case 0: return -v;
        case 1: return fabsf(v);
        case 2: return expf(v);
        case 3: return logf(v);
        case 4: return sqrtf(v);
        case 5: return tanhf(v);
        case 6: return 1.0f / (1.0f + expf(-v));
        case 7: {
            const float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
            return 0.5f * v * (1.0f + tanhf(inner));
        }
        default: return v / (1.0f + expf(-v));
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void unary_k(int op, const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    const int64_t n4 = VEC ? n / 4 : 0;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const float4 v = reinterpret_cast<const float4*>(x)[i];
        reinterpret_cast<float4*>(y)[i] = make_float4(una(op, v.x), una(op, v.y), una(op, v.z), una(op, v.w));
    }
    for (int64_t i = 4 * n4 + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        y[i] = una(op, x[i]);
}

// ---------------------------------------------------------------- reductions
// op: 0 sum, 1 mean, 2 max, 3 min.  Sums in double, max / min in float; NaN is skipped as the
// reference's `v > m` test skips it (fmax / fmin return the non-NaN operand).
struct Acc {
    double s;
    float m;
};

__device__ __forceinline__ Acc acc_init(int op) { return {0.0, op == 2 ? -INFINITY : INFINITY}; }
__device__ __forceinline__ void acc_add(int op, Acc& a, float v) {
    if (op <= 1) a.s += static_cast<double>(v);
    else if (op == 2) a.m = fmaxf(a.m, v);
    else a.m = fminf(a.m, v);
}
__device__ __forceinline__ void acc_merge(int op, Acc& a, const Acc& b) {
    if (op <= 1) a.s += b.s;
    else if (op == 2) a.m = fmaxf(a.m, b.m);
    else a.m = fminf(a.m, b.m);
}
__device__ __forceinline__ Acc wave_acc(int op, Acc a) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        Acc b;
        b.s = __shfl_xor(a.s, o, kWave);
        b.m = __shfl_xor(a.m, o, kWave);
        acc_merge(op, a, b);
    }
    return a;
}
// Block-wide reduction of 256 threads in a fixed order.
__device__ __forceinline__ Acc block_acc(int op, Acc a, Acc* red) {
    a = wave_acc(op, a);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    if (l == 0) red[w] = a;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int i = 1; i < static_cast<int>(blockDim.x / kWave); ++i) acc_merge(op, a, red[i]);
    return a;  // valid in thread 0
}

// Pass 1: block b reduces the contiguous chunk [b * chunk, (b + 1) * chunk).
__global__ __launch_bounds__(256) void reduce_part_k(int op, const float* __restrict__ x, int64_t n, int64_t chunk,
                                                     Acc* __restrict__ part) {
    __shared__ Acc red[4];
    const int64_t beg = static_cast<int64_t>(blockIdx.x) * chunk, end = beg + chunk < n ? beg + chunk : n;
    Acc a = acc_init(op);
    for (int64_t i = beg + threadIdx.x; i < end; i += blockDim.x) acc_add(op, a, x[i]);
    a = block_acc(op, a, red);
    if (threadIdx.x == 0) part[blockIdx.x] = a;
}

// Pass 2: one block over the partials; writes the scalar result.
__global__ __launch_bounds__(256) void reduce_final_k(int op, const Acc* __restrict__ part, int np, int64_t n,
                                                      float* __restrict__ out) {
    __shared__ Acc red[4];
    Acc a = acc_init(op);
    for (int i = threadIdx.x; i < np; i += blockDim.x) acc_merge(op, a, part[i]);
    a = block_acc(op, a, red);
    if (threadIdx.x == 0) {
        if (op == 0) out[0] = static_cast<float>(a.s);
        else if (op == 1) out[0] = static_cast<float>(a.s) / static_cast<float>(n);
        else out[0] = a.m;
    }
}

__device__ __forceinline__ float acc_out(int op, const Acc& a, int64_t rs) {
    if (op == 0) return static_cast<float>(a.s);
    if (op == 1) return static_cast<float>(a.s / static_cast<double>(rs));
    return a.m;
}

// Reduce the middle axis of [outer, rs, inner] with inner == 1: one wave per row.
__global__ __launch_bounds__(256) void reduce_rows_k(int op, const float* __restrict__ x, int64_t rows, int64_t rs,
                                                     float* __restrict__ out) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (row >= rows) return;
    const float* p = x + row * rs;
    Acc a = acc_init(op);
    for (int64_t k = threadIdx.x % kWave; k < rs; k += kWave) acc_add(op, a, p[k]);
    a = wave_acc(op, a);
    if (threadIdx.x % kWave == 0) out[row] = acc_out(op, a, rs);
}

// inner > 1: one thread per (outer, inner) output, consecutive threads on consecutive inner.
__global__ __launch_bounds__(256) void reduce_cols_k(int op, const float* __restrict__ x, int64_t outer, int64_t rs,
                                                     int64_t inner, float* __restrict__ out) {
    const int64_t total = outer * inner;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t o = i / inner, in = i % inner;
        const float* p = x + o * rs * inner + in;
        Acc a = acc_init(op);
        for (int64_t k = 0; k < rs; ++k) acc_add(op, a, p[k * inner]);
        out[i] = acc_out(op, a, rs);
    }
}

View make_view(int64_t offset, int ndim, const int64_t* shape, const int64_t* strides) {
    AIC_CHECK(ndim >= 0 && ndim <= kMaxDims, InvalidArgument, "tensor rank must be 0..", kMaxDims, ", got ", ndim);
    View v{};
    v.offset = offset;
    v.ndim = ndim;
    for (int d = 0; d < ndim; ++d) {
        AIC_CHECK(shape[d] >= 0, InvalidArgument, "negative dimension");
        v.shape[d] = shape[d];
        v.strides[d] = strides ? strides[d] : 0;
    }
    return v;
}

int64_t numel_of(int ndim, const int64_t* shape) {
    int64_t n = 1;
    for (int d = 0; d < ndim; ++d) n *= shape[d];
    return n;
}

bool contiguous(int ndim, const int64_t* shape, const int64_t* strides) {
    int64_t expect = 1;
    for (int d = ndim - 1; d >= 0; --d) {
        if (shape[d] == 0) return true;
        if (shape[d] != 1) {
            if (strides[d] != expect) return false;
            expect *= shape[d];
        }
    }
    return true;
}

}  // namespace

void strided_copy(const void* src, int64_t offset, int ndim, const int64_t* shape, const int64_t* strides,
                  int64_t elem_size, void* dst, hipStream_t s) {
    const View v = make_view(offset, ndim, shape, strides);
    AIC_CHECK(ndim == 0 || (shape && strides), InvalidArgument, "strided_copy: null shape or strides");
    const int64_t n = numel_of(ndim, shape);
    if (n == 0) return;
    AIC_CHECK(src && dst, InvalidArgument, "strided_copy: null pointer");
    if (contiguous(ndim, shape, strides)) {
        AIC_HIP_CHECK(hipMemcpyAsync(dst, static_cast<const char*>(src) + offset * elem_size,
                                     static_cast<size_t>(n * elem_size), hipMemcpyDeviceToDevice, s));
        return;
    }
    const dim3 grid(grid_for(n, 256)), block(256);
    switch (elem_size) {
        case 1: hipLaunchKernelGGL(strided_copy_k<uint8_t>, grid, block, 0, s, static_cast<const uint8_t*>(src), v, static_cast<uint8_t*>(dst), n); break;
        case 2: hipLaunchKernelGGL(strided_copy_k<uint16_t>, grid, block, 0, s, static_cast<const uint16_t*>(src), v, static_cast<uint16_t*>(dst), n); break;
        case 4: hipLaunchKernelGGL(strided_copy_k<uint32_t>, grid, block, 0, s, static_cast<const uint32_t*>(src), v, static_cast<uint32_t*>(dst), n); break;
        case 8: hipLaunchKernelGGL(strided_copy_k<uint64_t>, grid, block, 0, s, static_cast<const uint64_t*>(src), v, static_cast<uint64_t*>(dst), n); break;
        default: AIC_THROW(InvalidArgument, "strided_copy: element size must be 1, 2, 4 or 8, got ", elem_size);
    }
    AIC_LAUNCH_CHECK("strided_copy");
}

void cast(const void* src, DType from, void* dst, DType to, int64_t n, hipStream_t s) {
    AIC_CHECK(n >= 0, InvalidArgument, "cast: negative count");
    const int f = static_cast<int>(from), t = static_cast<int>(to);
    // the reference's table (src/tensor/tensor.cpp:392-407)
    const bool known = f == t || (f == 0 && t >= 1 && t <= 4) || (t == 0 && f >= 1 && f <= 4) || (f == 4 && t == 3) ||
                       (f == 3 && t == 4);
    AIC_CHECK(known, NotImplemented, "Type cast from ", dtype_name(from), " to ", dtype_name(to), " not implemented");
    if (n == 0) return;
    AIC_CHECK(src && dst, InvalidArgument, "cast: null pointer");
    if (f == t) {
        AIC_HIP_CHECK(hipMemcpyAsync(dst, src, static_cast<size_t>(n) * dtype_size(from), hipMemcpyDeviceToDevice, s));
        return;
    }
    const dim3 grid(grid_for(n, 256)), block(256);
#define AIC_CAST(F, T) \
    if (f == F && t == T) { hipLaunchKernelGGL((cast_k<F, T>), grid, block, 0, s, src, dst, n); AIC_LAUNCH_CHECK("cast"); return; }
    AIC_CAST(0, 1) AIC_CAST(0, 2) AIC_CAST(1, 0) AIC_CAST(2, 0) AIC_CAST(0, 4)
    AIC_CAST(4, 0) AIC_CAST(0, 3) AIC_CAST(3, 0) AIC_CAST(4, 3) AIC_CAST(3, 4)
#undef AIC_CAST
    AIC_THROW(NotImplemented, "Type cast from ", dtype_name(from), " to ", dtype_name(to), " not implemented");
}

void binary(int op, const float* a, int64_t a_off, int ra, const int64_t* a_shape, const int64_t* a_strides,
            const float* b, int64_t b_off, int rb, const int64_t* b_shape, const int64_t* b_strides, float* out,
            hipStream_t s) {
    AIC_CHECK(op >= 0 && op <= 3, InvalidArgument, "binary: unknown op ", op);
    AIC_CHECK(ra >= 0 && rb >= 0 && ra <= kMaxDims && rb <= kMaxDims, InvalidArgument, "binary: rank must be 0..8");
    // Shape::broadcast and Shape::broadcast_strides (src/core/shape.cpp:138-195)
    const int r = ra > rb ? ra : rb;
    int64_t oshape[kMaxDims], sa[kMaxDims], sb[kMaxDims];
    for (int i = 0; i < r; ++i) {
        const int ia = ra - 1 - i, ib = rb - 1 - i, io = r - 1 - i;
        const int64_t da = ia >= 0 ? a_shape[ia] : 1, db = ib >= 0 ? b_shape[ib] : 1;
        AIC_CHECK(da == db || da == 1 || db == 1, ShapeMismatch, "Cannot broadcast dimension ", da, " against ", db);
        oshape[io] = da > db ? da : db;
        sa[io] = (ia >= 0 && da == oshape[io]) ? a_strides[ia] : 0;
        sb[io] = (ib >= 0 && db == oshape[io]) ? b_strides[ib] : 0;
    }
    const int64_t n = numel_of(r, oshape);
    if (n == 0) return;
    AIC_CHECK(a && b && out, InvalidArgument, "binary: null pointer");
    const dim3 block(256);
    bool same = ra == rb;
    for (int i = 0; same && i < ra; ++i) same = a_shape[i] == b_shape[i];
    if (same && contiguous(ra, a_shape, a_strides) && contiguous(rb, b_shape, b_strides) &&
        reinterpret_cast<uintptr_t>(a + a_off) % 16 == 0 && reinterpret_cast<uintptr_t>(b + b_off) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(out) % 16 == 0) {
        hipLaunchKernelGGL(binary_flat_k, dim3(grid_for((n + 3) / 4, 256)), block, 0, s, op, a + a_off, b + b_off, out, n);
    } else {
        const View va = make_view(a_off, r, oshape, sa), vb = make_view(b_off, r, oshape, sb);
        hipLaunchKernelGGL(binary_bcast_k, dim3(grid_for(n, 256)), block, 0, s, op, a, va, b, vb, out, n);
    }
    AIC_LAUNCH_CHECK("binary");
}

void unary(int op, const float* x, float* y, int64_t n, hipStream_t s) {
    AIC_CHECK(op >= 0 && op <= 8, InvalidArgument, "unary: unknown op ", op);
    AIC_CHECK(n >= 0, InvalidArgument, "unary: negative count");
    if (n == 0) return;
    AIC_CHECK(x && y, InvalidArgument, "unary: null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0)
        hipLaunchKernelGGL(unary_k<true>, dim3(grid_for((n + 3) / 4, 256)), dim3(256), 0, s, op, x, y, n);
    else
        hipLaunchKernelGGL(unary_k<false>, dim3(grid_for(n, 256)), dim3(256), 0, s, op, x, y, n);
    AIC_LAUNCH_CHECK("unary");
}

void reduce_all(int op, const float* x, int64_t n, float* out, hipStream_t s) {
    AIC_CHECK(op >= 0 && op <= 3, InvalidArgument, "reduce: unknown op ", op);
    AIC_CHECK(n > 0 || op == 0, InvalidArgument, "Cannot reduce an empty tensor");
    AIC_CHECK((x || n == 0) && out, InvalidArgument, "reduce: null pointer");
    // about 16 K elements per block, at most 1024 blocks
    int64_t parts = (n + 16383) / 16384;
    if (parts < 1) parts = 1;
    if (parts > 1024) parts = 1024;
    const int64_t chunk = (n + parts - 1) / parts;
    Acc* part = static_cast<Acc*>(stream_scratch(sizeof(Acc) * static_cast<size_t>(parts), s));
    hipLaunchKernelGGL(reduce_part_k, dim3(static_cast<unsigned>(parts)), dim3(256), 0, s, op, x, n, chunk, part);
    hipLaunchKernelGGL(reduce_final_k, dim3(1), dim3(256), 0, s, op, part, static_cast<int>(parts), n, out);
    AIC_LAUNCH_CHECK("reduce_all");
}

void reduce_dim(int op, const float* x, int ndim, const int64_t* shape, int dim, float* out, hipStream_t s) {
    AIC_CHECK(op >= 0 && op <= 3, InvalidArgument, "reduce: unknown op ", op);
    AIC_CHECK(ndim >= 1 && ndim <= kMaxDims && shape, InvalidArgument, "reduce: rank must be 1..8");
    if (dim < 0) dim += ndim;
    AIC_CHECK(dim >= 0 && dim < ndim, OutOfRange, "Reduction dim out of range for rank ", ndim);
    const int64_t rs = shape[dim];
    AIC_CHECK(rs > 0, InvalidArgument, "Cannot reduce along dimension of size 0");
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < dim; ++i) outer *= shape[i];
    for (int i = dim + 1; i < ndim; ++i) inner *= shape[i];
    if (outer * inner == 0) return;
    AIC_CHECK(x && out, InvalidArgument, "reduce: null pointer");
    if (inner == 1)
        hipLaunchKernelGGL(reduce_rows_k, dim3(static_cast<unsigned>((outer + 3) / 4)), dim3(256), 0, s, op, x, outer, rs, out);
    else
        hipLaunchKernelGGL(reduce_cols_k, dim3(grid_for(outer * inner, 256)), dim3(256), 0, s, op, x, outer, rs, inner, out);
    AIC_LAUNCH_CHECK("reduce_dim");
}

void cat(const void* const* srcs, const int64_t* mids, int count, int64_t outer, int64_t inner, int64_t elem_size,
         void* dst, hipStream_t s) {
    AIC_CHECK(count >= 1 && srcs && mids && outer >= 0 && inner >= 0 && elem_size > 0, InvalidArgument, "cat: bad arguments");
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        AIC_CHECK(mids[i] >= 0, InvalidArgument, "cat: negative size");
        total += mids[i];
    }
    if (outer == 0 || inner == 0 || total == 0) return;
    AIC_CHECK(dst, InvalidArgument, "cat: null output");
    int64_t off = 0;
    for (int i = 0; i < count; ++i) {
        if (mids[i] > 0) {
            AIC_CHECK(srcs[i], InvalidArgument, "cat: null input ", i);
            const size_t w = static_cast<size_t>(mids[i] * inner * elem_size);
            AIC_HIP_CHECK(hipMemcpy2DAsync(static_cast<char*>(dst) + off * inner * elem_size,
                                           static_cast<size_t>(total * inner * elem_size), srcs[i], w, w,
                                           static_cast<size_t>(outer), hipMemcpyDeviceToDevice, s));
        }
        off += mids[i];
    }
}

void sum_to_shape(const float* g, int ndim, const int64_t* shape, int tr, const int64_t* target, float* out,
                  hipStream_t s) {
    AIC_CHECK(ndim >= 0 && ndim <= kMaxDims && tr >= 0 && tr <= ndim, InvalidArgument, "sum_to_shape: bad ranks");
    const int64_t n = numel_of(ndim, shape);
    AIC_CHECK(g && out, InvalidArgument, "sum_to_shape: null pointer");
    if (tr == 0) {
        reduce_all(0, g, n, out, s);
        return;
    }
    int64_t cur[kMaxDims];
    int r = ndim;
    for (int i = 0; i < ndim; ++i) cur[i] = shape[i];
    // the same sequence of per-dim sums as the reference, each rounded to float
    DeviceBuffer a, b;
    const float* src = g;
    int64_t cnt = n;
    auto step = [&](int dim) {
        const int64_t m = cnt / cur[dim];
        DeviceBuffer next(sizeof(float) * static_cast<size_t>(m > 0 ? m : 1), s);
        reduce_dim(0, src, r, cur, dim, next.as<float>(), s);
        a = std::move(b);
        b = std::move(next);
        src = b.as<float>();
        cnt = m;
    };
    while (r > tr) {
        step(0);
        for (int i = 0; i + 1 < r; ++i) cur[i] = cur[i + 1];
        --r;
    }
    for (int i = 0; i < tr; ++i)
        if (target[i] == 1 && cur[i] > 1) {
            step(i);
            cur[i] = 1;
        }
    for (int i = 0; i < tr; ++i)
        AIC_CHECK(cur[i] == target[i], ShapeMismatch, "sum_to_shape: gradient does not reduce to the target shape");
    if (cnt > 0) AIC_HIP_CHECK(hipMemcpyAsync(out, src, sizeof(float) * static_cast<size_t>(cnt), hipMemcpyDeviceToDevice, s));
}

}  // namespace aic::hip
