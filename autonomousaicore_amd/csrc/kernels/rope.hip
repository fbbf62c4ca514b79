// Rotary position embedding, half-split (NeoX) form, applied in place to the q and k
// column blocks of the projection output (no [B,H,S,hd] transpose is materialised).
// Replaces RotaryPositionEmbedding::forward / RoPEBackward (include/nn/rope.hpp:23-112),
// which slice, multiply, add and concatenate in six primitive ops per tensor.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

namespace aic::hip {

namespace {

template <typename T, int VN, bool INV>
__global__ __launch_bounds__(256) void rope_k(T* __restrict__ x, int64_t ldx, int64_t T_rows, int S, int heads, int hd,
                                              int64_t start_pos, const float* __restrict__ cos_t,
                                              const float* __restrict__ sin_t) {
    const int half = hd / 2;
    const int per_row = heads * (half / VN);
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= T_rows * per_row) return;
    const int64_t t = idx / per_row;
    const int r = static_cast<int>(idx % per_row);
    const int h = r / (half / VN);
    const int i0 = (r % (half / VN)) * VN;
    const int64_t pos = start_pos + (t % S);
    T* p1 = x + t * ldx + static_cast<int64_t>(h) * hd + i0;
    T* p2 = p1 + half;
    const float* c = cos_t + pos * half + i0;
    const float* sn = sin_t + pos * half + i0;
#pragma unroll
    for (int i = 0; i < VN; ++i) {
        const float a1 = ld(p1, i), a2 = ld(p2, i), cc = c[i], ss = sn[i];
        float o1, o2;
        if (!INV) {
            o1 = a1 * cc - a2 * ss;
            o2 = a1 * ss + a2 * cc;
        } else {
            o1 = a1 * cc + a2 * ss;
            o2 = a2 * cc - a1 * ss;
        }
        st(p1, i, o1);
        st(p2, i, o2);
    }
}

// Vector form: VN = 16 / sizeof(T) elements of each half per thread, one 16-byte load and store
// per half and 16-byte table reads.  Same per-element arithmetic as rope_k.
template <typename T, bool INV>
__global__ __launch_bounds__(256) void rope_v(T* __restrict__ x, int64_t ldx, int64_t T_rows, int S, int heads, int hd,
                                              int64_t start_pos, const float* __restrict__ cos_t,
                                              const float* __restrict__ sin_t) {
    constexpr int VN = 16 / sizeof(T);
    const int half = hd / 2;
    const int per_row = heads * (half / VN);
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= T_rows * per_row) return;
    const int64_t t = idx / per_row;
    const int r = static_cast<int>(idx % per_row);
    const int h = r / (half / VN);
    const int i0 = (r % (half / VN)) * VN;
    const int64_t pos = start_pos + (t % S);
    T* p1 = x + t * ldx + static_cast<int64_t>(h) * hd + i0;
    T* p2 = p1 + half;
    const float* c = cos_t + pos * half + i0;
    const float* sn = sin_t + pos * half + i0;
    float a1[VN], a2[VN], cc[VN], ss[VN], o1[VN], o2[VN];
    if constexpr (sizeof(T) == 2) {
        const uint4 u1 = *reinterpret_cast<const uint4*>(p1), u2 = *reinterpret_cast<const uint4*>(p2);
        const uint32_t w1[4] = {u1.x, u1.y, u1.z, u1.w}, w2[4] = {u2.x, u2.y, u2.z, u2.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            a1[2 * q] = __uint_as_float(w1[q] << 16);
            a1[2 * q + 1] = __uint_as_float(w1[q] & 0xffff0000u);
            a2[2 * q] = __uint_as_float(w2[q] << 16);
            a2[2 * q + 1] = __uint_as_float(w2[q] & 0xffff0000u);
        }
    } else {
        const float4 u1 = *reinterpret_cast<const float4*>(p1), u2 = *reinterpret_cast<const float4*>(p2);
        a1[0] = u1.x; a1[1] = u1.y; a1[2] = u1.z; a1[3] = u1.w;
        a2[0] = u2.x; a2[1] = u2.y; a2[2] = u2.z; a2[3] = u2.w;
    }
#pragma unroll
    for (int q = 0; q < VN; q += 4) {
        const float4 c4 = *reinterpret_cast<const float4*>(c + q), s4 = *reinterpret_cast<const float4*>(sn + q);
        cc[q] = c4.x; cc[q + 1] = c4.y; cc[q + 2] = c4.z; cc[q + 3] = c4.w;
        ss[q] = s4.x; ss[q + 1] = s4.y; ss[q + 2] = s4.z; ss[q + 3] = s4.w;
    }
#pragma unroll
    for (int i = 0; i < VN; ++i) {
        if (!INV) {
            o1[i] = a1[i] * cc[i] - a2[i] * ss[i];
            o2[i] = a1[i] * ss[i] + a2[i] * cc[i];
        } else {
            o1[i] = a1[i] * cc[i] + a2[i] * ss[i];
            o2[i] = a2[i] * cc[i] - a1[i] * ss[i];
        }
    }
    if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint4*>(p1) = make_uint4(pack_bf16x2(o1[0], o1[1]), pack_bf16x2(o1[2], o1[3]),
                                                   pack_bf16x2(o1[4], o1[5]), pack_bf16x2(o1[6], o1[7]));
        *reinterpret_cast<uint4*>(p2) = make_uint4(pack_bf16x2(o2[0], o2[1]), pack_bf16x2(o2[2], o2[3]),
                                                   pack_bf16x2(o2[4], o2[5]), pack_bf16x2(o2[6], o2[7]));
    } else {
        *reinterpret_cast<float4*>(p1) = make_float4(o1[0], o1[1], o1[2], o1[3]);
        *reinterpret_cast<float4*>(p2) = make_float4(o2[0], o2[1], o2[2], o2[3]);
    }
}

template <typename T>
void launch(void* x, int64_t ld, int64_t B, int64_t S, int64_t heads, int64_t hd, int64_t start_pos, const float* c,
            const float* sn, bool inverse, hipStream_t s) {
    const int64_t T_rows = B * S;
    const int half = static_cast<int>(hd / 2);
    constexpr int VV = 16 / sizeof(T);
    if (half % VV == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && (ld * sizeof(T)) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(c) % 16 == 0 && reinterpret_cast<uintptr_t>(sn) % 16 == 0) {
        const int64_t nv = T_rows * heads * (half / VV);
        const unsigned gv = static_cast<unsigned>((nv + 255) / 256);
        if (inverse)
            hipLaunchKernelGGL((rope_v<T, true>), dim3(gv), dim3(256), 0, s, static_cast<T*>(x), ld, T_rows,
                               static_cast<int>(S), static_cast<int>(heads), static_cast<int>(hd), start_pos, c, sn);
        else
            hipLaunchKernelGGL((rope_v<T, false>), dim3(gv), dim3(256), 0, s, static_cast<T*>(x), ld, T_rows,
                               static_cast<int>(S), static_cast<int>(heads), static_cast<int>(hd), start_pos, c, sn);
        AIC_LAUNCH_CHECK("rope");
        return;
    }
    const int VN = (half % 4 == 0) ? 4 : 1;
    const int64_t n = T_rows * heads * (half / VN);
    const unsigned grid = static_cast<unsigned>((n + 255) / 256);
    T* xp = static_cast<T*>(x);
#define AIC_ROPE(V, I)                                                                                        \
    hipLaunchKernelGGL((rope_k<T, V, I>), dim3(grid), dim3(256), 0, s, xp, ld, T_rows, static_cast<int>(S),     \
                       static_cast<int>(heads), static_cast<int>(hd), start_pos, c, sn)
    if (VN == 4) {
        if (inverse) AIC_ROPE(4, true); else AIC_ROPE(4, false);
    } else {
        if (inverse) AIC_ROPE(1, true); else AIC_ROPE(1, false);
    }
#undef AIC_ROPE
    AIC_LAUNCH_CHECK("rope");
}

}  // namespace

void rope(void* x, int64_t ld, int64_t B, int64_t S, int64_t heads, int64_t hd, int64_t start_pos, const float* cos_t,
          const float* sin_t, bool inverse, DType dt, hipStream_t s) {
    AIC_CHECK(hd > 0 && hd % 2 == 0, InvalidArgument, "rope: head_dim must be even, got ", hd);
    AIC_CHECK(B >= 0 && S >= 0 && heads > 0 && ld >= heads * hd && start_pos >= 0, InvalidArgument, "rope: bad shape");
    if (B * S == 0) return;
    if (dt == DType::Float32) launch<float>(x, ld, B, S, heads, hd, start_pos, cos_t, sin_t, inverse, s);
    else if (dt == DType::BFloat16) launch<bf16>(x, ld, B, S, heads, hd, start_pos, cos_t, sin_t, inverse, s);
    else AIC_THROW(DTypeMismatch, "rope: dtype must be f32 or bf16");
}

// Same float arithmetic as the reference's cache (include/nn/rope.hpp:122-144):
// freq_i = 1 / base^(2i/hd) in float, angle = float(pos) * freq_i, cos/sin in float.
void rope_tables_host(float* cos_t, float* sin_t, int64_t max_seq, int64_t hd, float base) {
    const int64_t half = hd / 2;
    for (int64_t i = 0; i < half; ++i) {
        const float exponent = static_cast<float>(2 * i) / static_cast<float>(hd);
        const float freq = 1.0f / std::pow(base, exponent);
        for (int64_t pos = 0; pos < max_seq; ++pos) {
            const float angle = static_cast<float>(pos) * freq;
            cos_t[pos * half + i] = std::cos(angle);
            sin_t[pos * half + i] = std::sin(angle);
        }
    }
}

}  // namespace aic::hip
