// RMSNorm forward/backward as single fused kernels (the reference builds RMSNorm from six
// primitive ops plus their backward nodes, include/nn/rms_norm.hpp:18-34).
// HBM-bound: one wave per row, 16-byte vector loads; the weight gradient is reduced
// per block into per-wave LDS slices and then across blocks in a fixed order
// (deterministic, no atomics).
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

template <typename T> struct Vec;
template <> struct Vec<float> { static constexpr int N = 4; };
template <> struct Vec<bf16> { static constexpr int N = 8; };

// Loads VN consecutive elements as fp32.
template <typename T, int VN>
__device__ __forceinline__ void load_vec(const T* p, float* out) {
    if constexpr (VN == 1) {
        out[0] = ld(p, 0);
    } else if constexpr (sizeof(T) == 4) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = __uint_as_float(w[i] << 16);
            out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
}
template <typename T, int VN>
__device__ __forceinline__ void store_vec(T* p, const float* in) {
    if constexpr (VN == 1) {
        st(p, 0, in[0]);
    } else if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(in[0], in[1], in[2], in[3]);
    } else {
        uint4 v;
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = static_cast<uint32_t>(f2bf_bits(in[2 * i])) | (static_cast<uint32_t>(f2bf_bits(in[2 * i + 1])) << 16);
        v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
        *reinterpret_cast<uint4*>(p) = v;
    }
}

template <typename T, int VN>
__global__ __launch_bounds__(256) void rmsnorm_fwd_k(const T* __restrict__ x, int64_t ldx, const float* __restrict__ w,
                                                     T* __restrict__ y, int64_t ldy, float* __restrict__ rms,
                                                     int64_t rows, int dim, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const T* xr = x + row * ldx;
    float ss = 0.0f;
    for (int j = lane * VN; j < dim; j += 64 * VN) {
        float v[VN];
        load_vec<T, VN>(xr + j, v);
#pragma unroll
        for (int i = 0; i < VN; ++i) ss += v[i] * v[i];
    }
    ss = wave_sum(ss);
    const float r = sqrtf(ss / static_cast<float>(dim) + eps);
    const float inv = 1.0f / r;
    if (lane == 0 && rms) rms[row] = r;
    T* yr = y + row * ldy;
    for (int j = lane * VN; j < dim; j += 64 * VN) {
        float v[VN], o[VN];
        load_vec<T, VN>(xr + j, v);
#pragma unroll
        for (int i = 0; i < VN; ++i) o[i] = (v[i] * inv) * w[j + i];
        store_vec<T, VN>(yr + j, o);
    }
}

// Register-resident forms for dim <= 64 * VN * CH: a lane holds its CH chunks of the row, so
// all of a row's loads are in flight at once and the row is read once.  Same arithmetic, in
// the same order, as the loop forms above and below (results are bit-identical).
template <typename T, int VN, int CH>
__global__ __launch_bounds__(256) void rmsnorm_fwd_r(const T* __restrict__ x, int64_t ldx, const float* __restrict__ w,
                                                     T* __restrict__ y, int64_t ldy, float* __restrict__ rms,
                                                     int64_t rows, int dim, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const T* xr = x + row * ldx;
    float v[CH][VN];
#pragma unroll
    for (int t = 0; t < CH; ++t) {
        const int c = (t * 64 + lane) * VN;
        if (c < dim) load_vec<T, VN>(xr + c, v[t]);
        else
#pragma unroll
            for (int i = 0; i < VN; ++i) v[t][i] = 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < CH; ++t)
#pragma unroll
        for (int i = 0; i < VN; ++i) ss += v[t][i] * v[t][i];
    ss = wave_sum(ss);
    const float r = sqrtf(ss / static_cast<float>(dim) + eps);
    const float inv = 1.0f / r;
    if (lane == 0 && rms) rms[row] = r;
    T* yr = y + row * ldy;
#pragma unroll
    for (int t = 0; t < CH; ++t) {
        const int c = (t * 64 + lane) * VN;
        if (c >= dim) continue;
        float o[VN];
#pragma unroll
        for (int i = 0; i < VN; ++i) o[i] = (v[t][i] * inv) * w[c + i];
        store_vec<T, VN>(yr + c, o);
    }
}

constexpr int kBwdRowsPerWave = 8;

// dx and per-block dw partials.  Block = 4 waves; wave w handles rows
// blockIdx*16 + w*4 .. +3.  dw partial of the block -> part[blockIdx][dim].
template <typename T, int VN>
__global__ __launch_bounds__(256) void rmsnorm_bwd_k(const T* __restrict__ dy, int64_t lddy, const T* __restrict__ x,
                                                     int64_t ldx, const float* __restrict__ w,
                                                     const float* __restrict__ rms, const T* dres, int64_t ldres,
                                                     T* dx, int64_t lddx, float* __restrict__ part, int64_t rows,
                                                     int dim) {
    extern __shared__ float sdw[];  // [4][dim] when part != nullptr
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (part)
        for (int j = threadIdx.x; j < 4 * dim; j += 256) sdw[j] = 0.0f;
    __syncthreads();
    for (int rr = 0; rr < kBwdRowsPerWave; ++rr) {
        const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kBwdRowsPerWave + rr;
        if (row >= rows) break;
        const T* gr = dy + row * lddy;
        const T* xr = x + row * ldx;
        const float r = rms[row];
        const float inv = 1.0f / r;
        float dot = 0.0f;
        for (int j = lane * VN; j < dim; j += 64 * VN) {
            float gv[VN], xv[VN];
            load_vec<T, VN>(gr + j, gv);
            load_vec<T, VN>(xr + j, xv);
#pragma unroll
            for (int i = 0; i < VN; ++i) dot += (gv[i] * w[j + i]) * xv[i];
        }
        dot = wave_sum(dot);
        const float coef = dot / (static_cast<float>(dim) * r * r * r);
        for (int j = lane * VN; j < dim; j += 64 * VN) {
            float gv[VN], xv[VN], o[VN];
            load_vec<T, VN>(gr + j, gv);
            load_vec<T, VN>(xr + j, xv);
            if (dres) {
                float rv[VN];
                load_vec<T, VN>(dres + row * ldres + j, rv);
#pragma unroll
                for (int i = 0; i < VN; ++i) o[i] = rv[i] + ((gv[i] * w[j + i]) * inv - xv[i] * coef);
            } else {
#pragma unroll
                for (int i = 0; i < VN; ++i) o[i] = (gv[i] * w[j + i]) * inv - xv[i] * coef;
            }
            if (part) {
#pragma unroll
                for (int i = 0; i < VN; ++i) sdw[wave * dim + j + i] += gv[i] * (xv[i] * inv);
            }
            store_vec<T, VN>(dx + row * lddx + j, o);
        }
    }
    if (!part) return;
    __syncthreads();
    for (int j = threadIdx.x; j < dim; j += 256)
        part[static_cast<int64_t>(blockIdx.x) * dim + j] = ((sdw[j] + sdw[dim + j]) + sdw[2 * dim + j]) + sdw[3 * dim + j];
}

// Register-resident backward: wave w of block b handles rows (4b + w) R .. (4b + w) R + R - 1
// (R = kBwdRegRowsPerWave, the loop form's count, so both write the same partial rows), with the
// next row's 16-byte chunks in flight while the current row is reduced and written (8 rows per
// wave with this prefetch: 13% faster than 4 without it at the 1B shape, half the partial rows);
// the lane's dw contributions accumulate in registers over its rows, then the four waves' sums
// are added in wave order, as the loop form does through LDS.
constexpr int kBwdRegRowsPerWave = 8;

template <typename T, int VN, int CH>
__global__ __launch_bounds__(256) void rmsnorm_bwd_r(const T* __restrict__ dy, int64_t lddy, const T* __restrict__ x,
                                                     int64_t ldx, const float* __restrict__ w,
                                                     const float* __restrict__ rms, const T* dres, int64_t ldres,
                                                     T* dx, int64_t lddx, float* __restrict__ part, int64_t rows,
                                                     int dim) {
    extern __shared__ float sdw[];  // [4][dim] when part != nullptr
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float wv[CH][VN], dwa[CH][VN];
#pragma unroll
    for (int t = 0; t < CH; ++t) {
        const int c = (t * 64 + lane) * VN;
#pragma unroll
        for (int i = 0; i < VN; ++i) {
            wv[t][i] = c < dim ? w[c + i] : 0.0f;
            dwa[t][i] = 0.0f;
        }
    }
    // the next row's 16-byte chunks are in flight while this row is reduced and written
    uint4 ng[CH], nx[CH], nr[CH];
    float nrm = 1.0f;
    auto fetch = [&](int64_t row) {
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            const int c = (t * 64 + lane) * VN;
            if (c < dim) {
                ng[t] = *reinterpret_cast<const uint4*>(dy + row * lddy + c);
                nx[t] = *reinterpret_cast<const uint4*>(x + row * ldx + c);
                nr[t] = dres ? *reinterpret_cast<const uint4*>(dres + row * ldres + c) : make_uint4(0, 0, 0, 0);
            } else {
                ng[t] = nx[t] = nr[t] = make_uint4(0, 0, 0, 0);
            }
        }
        nrm = rms[row];
    };
    auto unpack = [&](const uint4& u, float* o) {
        if constexpr (sizeof(T) == 4) {
            o[0] = __uint_as_float(u.x); o[1] = __uint_as_float(u.y);
            o[2] = __uint_as_float(u.z); o[3] = __uint_as_float(u.w);
        } else {
            const uint32_t q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[2 * i] = __uint_as_float(q[i] << 16);
                o[2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
            }
        }
    };
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kBwdRegRowsPerWave;
    if (row0 < rows) fetch(row0);
    for (int rr = 0; rr < kBwdRegRowsPerWave; ++rr) {
        const int64_t row = row0 + rr;
        if (row >= rows) break;
        uint4 cg[CH], cx[CH], cr[CH];
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            cg[t] = ng[t];
            cx[t] = nx[t];
            cr[t] = nr[t];
        }
        const float r = nrm;
        if (rr + 1 < kBwdRegRowsPerWave && row + 1 < rows) fetch(row + 1);
        float gv[CH][VN], xv[CH][VN];
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            unpack(cg[t], gv[t]);
            unpack(cx[t], xv[t]);
        }
        const float inv = 1.0f / r;
        float dot = 0.0f;
#pragma unroll
        for (int t = 0; t < CH; ++t)
#pragma unroll
            for (int i = 0; i < VN; ++i) dot += (gv[t][i] * wv[t][i]) * xv[t][i];
        dot = wave_sum(dot);
        const float coef = dot / (static_cast<float>(dim) * r * r * r);
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            const int c = (t * 64 + lane) * VN;
            if (c >= dim) continue;
            float rv[VN], o[VN];
            unpack(cr[t], rv);
#pragma unroll
            for (int i = 0; i < VN; ++i) {
                const float g = (gv[t][i] * wv[t][i]) * inv - xv[t][i] * coef;
                o[i] = dres ? rv[i] + g : g;
                if (part) dwa[t][i] += gv[t][i] * (xv[t][i] * inv);
            }
            store_vec<T, VN>(dx + row * lddx + c, o);
        }
    }
    if (!part) return;
#pragma unroll
    for (int t = 0; t < CH; ++t) {
        const int c = (t * 64 + lane) * VN;
        if (c < dim)
#pragma unroll
            for (int i = 0; i < VN; ++i) sdw[wave * dim + c + i] = dwa[t][i];
    }
    __syncthreads();
    for (int j = threadIdx.x; j < dim; j += 256)
        part[static_cast<int64_t>(blockIdx.x) * dim + j] = ((sdw[j] + sdw[dim + j]) + sdw[2 * dim + j]) + sdw[3 * dim + j];
}

// dw = sum of the per-block partials, 8 columns per block so the whole chip takes part: thread t
// adds partials t, t + 256, ... of its column pair in order, then a fixed-order block tree.
__device__ __forceinline__ void reduce_parts8_body(const float* __restrict__ part, int nparts, int dim, float* dw,
                                                   int accumulate, int c0) {
    __shared__ float red[256][9];
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    // four partial rows' loads in flight per thread, added in order
    for (int b0 = threadIdx.x; b0 < nparts; b0 += 4 * 256) {
        float4 u[4], v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int b = b0 + k * 256;
            if (b < nparts) {
                u[k] = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(b) * dim + c0);
                v[k] = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(b) * dim + c0 + 4);
            } else {
                u[k] = v[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            acc[0] += u[k].x; acc[1] += u[k].y; acc[2] += u[k].z; acc[3] += u[k].w;
            acc[4] += v[k].x; acc[5] += v[k].y; acc[6] += v[k].z; acc[7] += v[k].w;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) red[threadIdx.x][i] = acc[i];
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (threadIdx.x < h)
#pragma unroll
            for (int i = 0; i < 8; ++i) red[threadIdx.x][i] += red[threadIdx.x + h][i];
        __syncthreads();
    }
    if (threadIdx.x < 8) {
        const int j = c0 + threadIdx.x;
        dw[j] = accumulate ? dw[j] + red[0][threadIdx.x] : red[0][threadIdx.x];
    }
}

__global__ __launch_bounds__(256) void reduce_parts8_k(const float* __restrict__ part, int nparts, int dim,
                                                       float* dw, int accumulate) {
    reduce_parts8_body(part, nparts, dim, dw, accumulate, blockIdx.x * 8);
}

// reduce_parts8_k for several norms at once: blockIdx.y = norm t, with its partial rows and dw.
constexpr int kDwBatch = 64;
struct DwBatch {
    const float* part[kDwBatch];
    float* dw[kDwBatch];
};
__global__ __launch_bounds__(256) void reduce_parts8_batch_k(const DwBatch b, int nparts, int dim) {
    reduce_parts8_body(b.part[blockIdx.y], nparts, dim, b.dw[blockIdx.y], 0, blockIdx.x * 8);
}

// dw[j] = sum over partial rows b of part[b][j], in a fixed order: block = 64 columns x 16
// waves, wave w sums rows w, w+16, ...; the 16 wave sums are then added in wave order.
__global__ __launch_bounds__(1024) void reduce_parts_k(const float* __restrict__ part, int nparts, int dim, float* dw,
                                                       int accumulate) {
    __shared__ float red[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + lane;
    float s = 0.0f;
    if (j < dim)
        for (int b = wave; b < nparts; b += 16) s += part[static_cast<int64_t>(b) * dim + j];
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && j < dim) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; ++w) t += red[w][lane];
        dw[j] = accumulate ? dw[j] + t : t;
    }
}

// Chunks of vn elements per lane for a row of dim, rounded up to a power of two (0: too long
// for the register forms).
int chunks_for(int64_t dim, int vn) {
    const int64_t need = (dim + 64 * vn - 1) / (64 * vn);
    for (int c = 1; c <= 8; c *= 2)
        if (need <= c) return c;
    return 0;
}

bool vec_ok(const void* p, int64_t ld, int64_t dim, int vn, size_t es) {
    return (reinterpret_cast<uintptr_t>(p) % (vn * es)) == 0 && ld % vn == 0 && dim % vn == 0;
}

template <typename T>
void fwd_t(const void* x, int64_t ldx, const float* w, void* y, int64_t ldy, float* rms, int64_t rows, int64_t dim,
           float eps, hipStream_t s) {
    constexpr int VN = Vec<T>::N;
    const unsigned grid = static_cast<unsigned>((rows + 3) / 4);
    const int ch = chunks_for(dim, VN);
    const bool vec = vec_ok(x, ldx, dim, VN, sizeof(T)) && vec_ok(y, ldy, dim, VN, sizeof(T));
#define AIC_FWD_R(CH)                                                                                            \
    hipLaunchKernelGGL((rmsnorm_fwd_r<T, VN, CH>), dim3(grid), dim3(256), 0, s, static_cast<const T*>(x), ldx, w, \
                       static_cast<T*>(y), ldy, rms, rows, static_cast<int>(dim), eps)
    if (vec && ch == 1) AIC_FWD_R(1);
    else if (vec && ch == 2) AIC_FWD_R(2);
    else if (vec && ch == 4) AIC_FWD_R(4);
    else if (vec && ch == 8) AIC_FWD_R(8);
#undef AIC_FWD_R
    else if (vec)
        hipLaunchKernelGGL((rmsnorm_fwd_k<T, VN>), dim3(grid), dim3(256), 0, s, static_cast<const T*>(x), ldx, w,
                           static_cast<T*>(y), ldy, rms, rows, static_cast<int>(dim), eps);
    else
        hipLaunchKernelGGL((rmsnorm_fwd_k<T, 1>), dim3(grid), dim3(256), 0, s, static_cast<const T*>(x), ldx, w,
                           static_cast<T*>(y), ldy, rms, rows, static_cast<int>(dim), eps);
    AIC_LAUNCH_CHECK("rmsnorm_fwd");
}

template <typename T>
void bwd_t(const void* dy, int64_t lddy, const void* x, int64_t ldx, const float* w, const float* rms,
           const void* dres, int64_t ldres, void* dx, int64_t lddx, float* dw, bool accumulate, int64_t rows,
           int64_t dim, hipStream_t s, float* ext_part = nullptr) {
    constexpr int VN = Vec<T>::N;
    const bool vec = vec_ok(dy, lddy, dim, VN, sizeof(T)) && vec_ok(x, ldx, dim, VN, sizeof(T)) &&
                     vec_ok(dx, lddx, dim, VN, sizeof(T)) && (!dres || vec_ok(dres, ldres, dim, VN, sizeof(T)));
    const int ch = chunks_for(dim, VN);
    const bool reg = vec && ch > 0;
    const int64_t rows_per_block = 4 * (reg ? kBwdRegRowsPerWave : kBwdRowsPerWave);
    const unsigned grid = static_cast<unsigned>((rows + rows_per_block - 1) / rows_per_block);
    float* part = ext_part;  // the caller's partial rows (reduced later), or scratch reduced below
    if (dw && !part) part = static_cast<float*>(stream_scratch(sizeof(float) * grid * dim, s));
    const size_t lds = dw ? sizeof(float) * 4 * dim : 0;
    AIC_CHECK(lds <= 160 * 1024, InvalidArgument, "rmsnorm_bwd: dim too large for the LDS weight-gradient slices");
#define AIC_BWD_R(CH)                                                                                         \
    hipLaunchKernelGGL((rmsnorm_bwd_r<T, VN, CH>), dim3(grid), dim3(256), lds, s, static_cast<const T*>(dy), \
                       lddy, static_cast<const T*>(x), ldx, w, rms, static_cast<const T*>(dres), ldres,        \
                       static_cast<T*>(dx), lddx, part, rows, static_cast<int>(dim))
    if (vec && ch == 1) AIC_BWD_R(1);
    else if (vec && ch == 2) AIC_BWD_R(2);
    else if (vec && ch == 4) AIC_BWD_R(4);
    else if (vec && ch == 8) AIC_BWD_R(8);
#undef AIC_BWD_R
    else if (vec)
        hipLaunchKernelGGL((rmsnorm_bwd_k<T, VN>), dim3(grid), dim3(256), lds, s, static_cast<const T*>(dy), lddy,
                           static_cast<const T*>(x), ldx, w, rms, static_cast<const T*>(dres), ldres,
                           static_cast<T*>(dx), lddx, part, rows, static_cast<int>(dim));
    else
        hipLaunchKernelGGL((rmsnorm_bwd_k<T, 1>), dim3(grid), dim3(256), lds, s, static_cast<const T*>(dy), lddy,
                           static_cast<const T*>(x), ldx, w, rms, static_cast<const T*>(dres), ldres,
                           static_cast<T*>(dx), lddx, part, rows, static_cast<int>(dim));
    AIC_LAUNCH_CHECK("rmsnorm_bwd");
    if (dw && !ext_part) {
        if (dim % 8 == 0)
            hipLaunchKernelGGL(reduce_parts8_k, dim3(static_cast<unsigned>(dim / 8)), dim3(256), 0, s, part,
                               static_cast<int>(grid), static_cast<int>(dim), dw, accumulate ? 1 : 0);
        else
            hipLaunchKernelGGL(reduce_parts_k, dim3(static_cast<unsigned>((dim + 63) / 64)), dim3(1024), 0, s, part,
                               static_cast<int>(grid), static_cast<int>(dim), dw, accumulate ? 1 : 0);
        AIC_LAUNCH_CHECK("rmsnorm_bwd reduce");
    }
}

}  // namespace

void rmsnorm_fwd(const void* x, int64_t ldx, const float* w, void* y, int64_t ldy, float* rms, int64_t rows,
                 int64_t dim, float eps, DType dt, hipStream_t s) {
    AIC_CHECK(rows >= 0 && dim > 0 && ldx >= dim && ldy >= dim, InvalidArgument, "rmsnorm_fwd: bad shape");
    if (rows == 0) return;
    if (dt == DType::Float32) fwd_t<float>(x, ldx, w, y, ldy, rms, rows, dim, eps, s);
    else if (dt == DType::BFloat16) fwd_t<bf16>(x, ldx, w, y, ldy, rms, rows, dim, eps, s);
    else AIC_THROW(DTypeMismatch, "rmsnorm_fwd: dtype must be f32 or bf16");
}

static_assert(kBwdRowsPerWave == kBwdRegRowsPerWave, "both backward forms take the same rows per block");

int64_t rmsnorm_bwd_part_rows(int64_t rows) { return (rows + 4 * kBwdRowsPerWave - 1) / (4 * kBwdRowsPerWave); }

void rmsnorm_bwd_deferred(const void* dy, int64_t lddy, const void* x, int64_t ldx, const float* w, const float* rms,
                          const void* dres, int64_t ldres, void* dx, int64_t lddx, float* part, int64_t rows,
                          int64_t dim, DType dt, hipStream_t s) {
    AIC_CHECK(rows > 0 && dim > 0 && dim % 8 == 0 && lddy >= dim && ldx >= dim && lddx >= dim && part,
              InvalidArgument, "rmsnorm_bwd_deferred: bad shape");
    if (dt == DType::Float32)
        bwd_t<float>(dy, lddy, x, ldx, w, rms, dres, ldres, dx, lddx, part, false, rows, dim, s, part);
    else if (dt == DType::BFloat16)
        bwd_t<bf16>(dy, lddy, x, ldx, w, rms, dres, ldres, dx, lddx, part, false, rows, dim, s, part);
    else AIC_THROW(DTypeMismatch, "rmsnorm_bwd_deferred: dtype must be f32 or bf16");
}

void rmsnorm_dw_reduce(const float* const* parts, float* const* dws, int count, int64_t rows, int64_t dim,
                       hipStream_t s) {
    AIC_CHECK(count >= 0 && rows > 0 && dim > 0 && dim % 8 == 0, InvalidArgument, "rmsnorm_dw_reduce: bad shape");
    const int nparts = static_cast<int>(rmsnorm_bwd_part_rows(rows));
    for (int t0 = 0; t0 < count; t0 += kDwBatch) {
        DwBatch b;
        const int n = std::min(count - t0, kDwBatch);
        for (int i = 0; i < kDwBatch; ++i) {
            b.part[i] = parts[t0 + std::min(i, n - 1)];
            b.dw[i] = dws[t0 + std::min(i, n - 1)];
        }
        hipLaunchKernelGGL(reduce_parts8_batch_k, dim3(static_cast<unsigned>(dim / 8), static_cast<unsigned>(n)),
                           dim3(256), 0, s, b, nparts, static_cast<int>(dim));
        AIC_LAUNCH_CHECK("rmsnorm_dw_reduce");
    }
}

void rmsnorm_bwd(const void* dy, int64_t lddy, const void* x, int64_t ldx, const float* w, const float* rms,
                 const void* dres, int64_t ldres, void* dx, int64_t lddx, float* dw, bool accumulate, int64_t rows,
                 int64_t dim, DType dt, hipStream_t s) {
    AIC_CHECK(rows >= 0 && dim > 0 && lddy >= dim && ldx >= dim && lddx >= dim, InvalidArgument,
              "rmsnorm_bwd: bad shape");
    if (rows == 0) return;
    if (dt == DType::Float32) bwd_t<float>(dy, lddy, x, ldx, w, rms, dres, ldres, dx, lddx, dw, accumulate, rows, dim, s);
    else if (dt == DType::BFloat16)
        bwd_t<bf16>(dy, lddy, x, ldx, w, rms, dres, ldres, dx, lddx, dw, accumulate, rows, dim, s);
    else AIC_THROW(DTypeMismatch, "rmsnorm_bwd: dtype must be f32 or bf16");
}

}  // namespace aic::hip
