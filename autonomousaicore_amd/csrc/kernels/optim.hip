// Optimizer tail of the training step, kept entirely on the device:
//   grad_sqnorm_multi  global sum of squares (fp64 partials, fixed-order final reduction)
//                      fused with the non-finite scan of the loss scaler
//   optim_finalize     one thread: loss-scaler skip/backoff/growth + clip coefficient
//   adamw_multi        fused AdamW (+ bf16 shadow copy of the updated weights)
// Replaces clip_grad_norm_ (src/optim/clip_grad.cpp:11-53, one host sync per parameter on
// the GPU path), DynamicLossScaler::unscale_and_update (src/train/amp.cpp:68-152,
// cudaMalloc + sync per parameter) and cuda_adamw_step (src/cuda/cuda_adamw.cu:22-89,
// one launch per parameter).  No host synchronisation is needed between backward and the
// update.
#include <cmath>
#include <mutex>

#include "../../../include/aic_hip.h"
#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

constexpr int kNormBlocks = 1024;

__device__ __forceinline__ bool finite_(float x) { return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u; }

// Block `bid` of `nb` blocks over the tensor g[0..n): its partial sum of squares and non-finite flag.
__device__ __forceinline__ void sqnorm_block(const float* __restrict__ g, int64_t n, int bid, int nb, double* part,
                                             int* part_nf) {
    __shared__ double sd[256];
    __shared__ int sn[256];
    double acc = 0.0;
    int nf = 0;
    const int64_t n4 = ((reinterpret_cast<uintptr_t>(g) & 15u) == 0) ? n / 4 : 0;
    const float4* g4 = reinterpret_cast<const float4*>(g);
    const int64_t stride = static_cast<int64_t>(nb) * 256;
    int64_t i = static_cast<int64_t>(bid) * 256 + threadIdx.x;
    // four loads in flight per thread; the values are added in the same order as one at a time
    for (; i + 3 * stride < n4; i += 4 * stride) {
        f32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g4) + i + u * stride);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            nf |= !finite_(v[u].x) | !finite_(v[u].y) | !finite_(v[u].z) | !finite_(v[u].w);
            acc += static_cast<double>(v[u].x * v[u].x + v[u].y * v[u].y) +
                   static_cast<double>(v[u].z * v[u].z + v[u].w * v[u].w);
        }
    }
    for (; i < n4; i += stride) {
        const float4 v = g4[i];
        nf |= !finite_(v.x) | !finite_(v.y) | !finite_(v.z) | !finite_(v.w);
        acc += static_cast<double>(v.x * v.x + v.y * v.y) + static_cast<double>(v.z * v.z + v.w * v.w);
    }
    for (int64_t i = n4 * 4 + static_cast<int64_t>(bid) * 256 + threadIdx.x; i < n; i += stride) {
        const float v = g[i];
        nf |= !finite_(v);
        acc += static_cast<double>(v) * static_cast<double>(v);
    }
    sd[threadIdx.x] = acc;
    sn[threadIdx.x] = nf;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            sd[threadIdx.x] += sd[threadIdx.x + o];
            sn[threadIdx.x] |= sn[threadIdx.x + o];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        part[bid] = sd[0];
        part_nf[bid] = sn[0];
    }
}

__global__ __launch_bounds__(256) void sqnorm_k(const float* __restrict__ g, int64_t n, double* part, int* part_nf) {
    sqnorm_block(g, n, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), part, part_nf);
}

// Several tensors' sqnorm_k blocks in one launch: tensor t owns the blocks [first[t], first[t+1])
// and its partials land at part + first[t], exactly as one sqnorm_k launch per tensor.
constexpr int kSqMultiMax = 128;
struct SqMulti {
    const float* g[kSqMultiMax];
    int64_t n[kSqMultiMax];
    int first[kSqMultiMax + 1];
    int count;
};
__global__ __launch_bounds__(256) void sqnorm_multi_k(const SqMulti m, double* part, int* part_nf) {
    const int b = static_cast<int>(blockIdx.x);
    int t = 0;
    while (t + 1 < m.count && b >= m.first[t + 1]) ++t;
    const int f0 = m.first[t];
    sqnorm_block(m.g[t], m.n[t], b - f0, m.first[t + 1] - f0, part + f0, part_nf + f0);
}

__global__ __launch_bounds__(1024) void sqnorm_final_k(const double* __restrict__ part, const int* __restrict__ part_nf,
                                                       int nparts, double* out, int* out_nf) {
    __shared__ double sd[1024];
    __shared__ int sn[1024];
    double acc = 0.0;
    int nf = 0;
    for (int i = threadIdx.x; i < nparts; i += 1024) {
        acc += part[i];
        nf |= part_nf[i];
    }
    sd[threadIdx.x] = acc;
    sn[threadIdx.x] = nf;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            sd[threadIdx.x] += sd[threadIdx.x + o];
            sn[threadIdx.x] |= sn[threadIdx.x + o];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        *out = sd[0];
        *out_nf = sn[0];
    }
}

// First level of the sum of many partial slots: block b adds slots [4096 b, 4096 (b + 1)), four
// per thread in order, then a fixed tree; the second level is sqnorm_final_k over the blocks.
__global__ __launch_bounds__(1024) void sqsum_level1_k(const double* __restrict__ part, const int* __restrict__ part_nf,
                                                       int64_t n, double* out, int* out_nf) {
    __shared__ double sd[1024];
    __shared__ int sn[1024];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * 4096;
    double v[4];
    int f[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t i = base + u * 1024 + threadIdx.x;
        v[u] = i < n ? part[i] : 0.0;
        f[u] = i < n ? part_nf[i] : 0;
    }
    sd[threadIdx.x] = ((v[0] + v[1]) + v[2]) + v[3];
    sn[threadIdx.x] = f[0] | f[1] | f[2] | f[3];
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            sd[threadIdx.x] += sd[threadIdx.x + o];
            sn[threadIdx.x] |= sn[threadIdx.x + o];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        out[blockIdx.x] = sd[0];
        out_nf[blockIdx.x] = sn[0];
    }
}
// Zeroes n gradient-norm slots (fp64 partials, then int flags).
__global__ __launch_bounds__(256) void sqslot_clear_k(double* part, int* part_nf, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        part[i] = 0.0;
        part_nf[i] = 0;
    }
}
__global__ void scale_k(float* g, int64_t n, const float* scale) {
    const float s = *scale;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        g[i] *= s;
}

// DynamicLossScaler::unscale_and_update (src/train/amp.cpp:118-152), then clip_grad_norm_
// (src/optim/clip_grad.cpp:40-50), folded into one multiplier for AdamW.
__global__ void finalize_k(const double* sqnorm, const int* nonfinite, aic_optim_ctl* c) {
    const float scale = c->use_scaler ? c->scale : 1.0f;
    if (c->use_scaler && *nonfinite) {
        c->skip = 1;
        c->scale = fmaxf(c->min_scale, c->scale * c->backoff_factor);
        c->good_steps = 0;
        c->skipped_steps += 1;
        c->grad_norm = NAN;
        c->grad_mult = 0.0f;
        return;
    }
    c->skip = 0;
    const float inv = 1.0f / scale;
    const float norm = static_cast<float>(sqrt(*sqnorm) * static_cast<double>(inv));
    c->grad_norm = norm;
    float mult = inv;
    if (c->max_grad_norm > 0.0f) {
        const float coef = c->max_grad_norm / (norm + 1e-6f);
        if (coef < 1.0f) mult = inv * coef;
    }
    c->grad_mult = mult;
    c->step += 1;
    if (c->use_scaler) {
        c->good_steps += 1;
        if (c->good_steps >= c->growth_interval) {
            c->scale = fminf(c->max_scale, c->scale * c->growth_factor);
            c->good_steps = 0;
        }
    }
}

template <bool BF16COPY>
__global__ __launch_bounds__(256) void adamw_k(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                                               float* __restrict__ v, bf16* __restrict__ pb, int64_t n, float lr,
                                               float beta1, float beta2, float eps, float wd, int64_t host_step,
                                               float host_bc1, float host_bc2, const aic_optim_ctl* __restrict__ ctl) {
    // bias corrections: from the device step count (ctl), from a host step count, or as
    // given by the caller (host_step == 0), which is how AdamW::step passes them
    float mult = 1.0f;
    int64_t step = host_step;
    if (ctl) {
        if (ctl->skip) return;
        mult = ctl->grad_mult;
        step = ctl->step;
    }
    const float bc1 = step > 0 ? 1.0f - powf(beta1, static_cast<float>(step)) : host_bc1;
    const float bc2 = step > 0 ? 1.0f - powf(beta2, static_cast<float>(step)) : host_bc2;
    const float ob1 = 1.0f - beta1, ob2 = 1.0f - beta2, lrwd = lr * wd;
    const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(m) |
                       reinterpret_cast<uintptr_t>(v)) & 15u) == 0 &&
                     (!BF16COPY || (reinterpret_cast<uintptr_t>(pb) & 7u) == 0);
    const int64_t n4 = vec ? n / 4 : 0;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    // Streaming pass: two float4 groups per thread per iteration (8 loads in flight), all
    // accesses non-temporal, since nothing here is read again before the next step.
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * blockDim.x * 2 + threadIdx.x; base < n4; base += 2 * stride) {
        f32x4 pp[2], gg[2], mm[2], vv[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t i = base + u * blockDim.x;
            if (i < n4) {
                pp[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + i);
                gg[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g) + i);
                mm[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(m) + i);
                vv[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(v) + i);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t i = base + u * blockDim.x;
            if (i >= n4) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float gr = gg[u][j] * mult;
                float par = pp[u][j];
                par -= lrwd * par;
                const float m1 = beta1 * mm[u][j] + ob1 * gr;
                const float v1 = beta2 * vv[u][j] + ob2 * gr * gr;
                mm[u][j] = m1;
                vv[u][j] = v1;
                par -= lr * ((m1 / bc1) / (sqrtf(v1 / bc2) + eps));
                pp[u][j] = par;
            }
            __builtin_nontemporal_store(pp[u], reinterpret_cast<f32x4*>(p) + i);
            __builtin_nontemporal_store(mm[u], reinterpret_cast<f32x4*>(m) + i);
            __builtin_nontemporal_store(vv[u], reinterpret_cast<f32x4*>(v) + i);
            if (BF16COPY) {
                u32x2 w;
                w[0] = static_cast<uint32_t>(f2bf_bits(pp[u][0])) | (static_cast<uint32_t>(f2bf_bits(pp[u][1])) << 16);
                w[1] = static_cast<uint32_t>(f2bf_bits(pp[u][2])) | (static_cast<uint32_t>(f2bf_bits(pp[u][3])) << 16);
                __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(pb) + i);
            }
        }
    }
    for (int64_t i = n4 * 4 + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float gr = g[i] * mult;
        float par = p[i];
        par -= lrwd * par;
        const float m1 = beta1 * m[i] + ob1 * gr;
        const float v1 = beta2 * v[i] + ob2 * gr * gr;
        m[i] = m1;
        v[i] = v1;
        par -= lr * ((m1 / bc1) / (sqrtf(v1 / bc2) + eps));
        p[i] = par;
        if (BF16COPY) pb[i] = f2bf(par);
    }
}

__global__ void cast_k(const float* __restrict__ src, bf16* __restrict__ dst, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        dst[i] = f2bf(src[i]);
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__global__ void fill_normal_k(float* dst, int64_t n, uint64_t seed, uint64_t offset, float mean, float std) {
    const uint64_t key = splitmix64(seed);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const uint64_t c = offset + static_cast<uint64_t>(i);
        const uint64_t r1 = splitmix64(key ^ (2 * c)), r2 = splitmix64(key ^ (2 * c + 1));
        const double u1 = (static_cast<double>(r1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        const double u2 = static_cast<double>(r2 >> 11) * (1.0 / 9007199254740992.0);
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        dst[i] = mean + std * static_cast<float>(z);
    }
}

__global__ void fill_const_k(float* dst, int64_t n, float v) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        dst[i] = v;
}

}  // namespace

namespace {

constexpr int kMaxNormTensors = 4096;

// Blocks of sqnorm_k per tensor (one fp64 partial and one flag each); returns the total.
int64_t sqnorm_blocks(const int64_t* sizes, int count, int* blocks) {
    int64_t total = 0;
    for (int t = 0; t < count; ++t) {
        AIC_CHECK(sizes[t] >= 0, InvalidArgument, "grad_sqnorm_multi: negative size of tensor ", t);
        const int64_t nb = (sizes[t] + 256 * 16 - 1) / (256 * 16);
        blocks[t] = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(nb, kNormBlocks)));
        total += blocks[t];
    }
    return total;
}

// pd: max(total, 1) fp64 partials; pn: as many int flags.
void sqnorm_launch(const float* const* grads, const int64_t* sizes, int count, const int* blocks, int total,
                   double* pd, int* pn, double* sqnorm, int* nonfinite, hipStream_t s) {
    int off = 0;
    for (int t = 0; t < count; ++t) {
        hipLaunchKernelGGL(sqnorm_k, dim3(blocks[t]), dim3(256), 0, s, grads[t], sizes[t], pd + off, pn + off);
        AIC_LAUNCH_CHECK("grad_sqnorm");
        off += blocks[t];
    }
    hipLaunchKernelGGL(sqnorm_final_k, dim3(1), dim3(1024), 0, s, pd, pn, total, sqnorm, nonfinite);
    AIC_LAUNCH_CHECK("grad_sqnorm_final");
}

}  // namespace

void grad_sqnorm_multi(const float* const* grads, const int64_t* sizes, int count, double* sqnorm, int* nonfinite,
                       hipStream_t s) {
    AIC_CHECK(count >= 0 && sqnorm && nonfinite, InvalidArgument, "grad_sqnorm_multi: bad arguments");
    AIC_CHECK(count <= kMaxNormTensors, InvalidArgument, "grad_sqnorm_multi: at most ", kMaxNormTensors, " tensors");
    int blocks[kMaxNormTensors];
    const int total = static_cast<int>(sqnorm_blocks(sizes, count, blocks));
    double* pd = static_cast<double*>(
        stream_scratch(sizeof(double) * std::max(total, 1) + sizeof(int) * std::max(total, 1), s));
    int* pn = reinterpret_cast<int*>(pd + std::max(total, 1));
    sqnorm_launch(grads, sizes, count, blocks, total, pd, pn, sqnorm, nonfinite, s);
}

// ---------------------------------------------------------------------------------------
// Allocation-free grad_sqnorm_multi.  The per-block partials live in `scratch`, a file-scope
// device array (each device holds its own copy until the process ends): fp64 partials in
// the first kNoAllocMaxBlocks slots, then the int non-finite flags.  Host code never passes
// the array's name to a kernel (on the host it is only a stand-in for the symbol); the
// device address comes from hipGetSymbolAddress, once per device, on the first call with
// that device current.  Every block overwrites its own partial, so nothing has to be
// cleared between calls; calls that overlap on one device race on the array.
// ---------------------------------------------------------------------------------------
constexpr int64_t kNoAllocMaxBlocks = int64_t{1} << 17;  // 1.5 MiB in total
static __device__ __align__(256) double scratch[kNoAllocMaxBlocks + kNoAllocMaxBlocks / 2];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

double* device_scratch() {
    int dev = 0;
    AIC_HIP_CHECK(hipGetDevice(&dev));
    AIC_CHECK(dev >= 0 && dev < kMaxDevices, InvalidArgument, "grad_sqnorm_multi_noalloc: device ", dev,
              " beyond the ", kMaxDevices, " supported");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        AIC_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        AIC_CHECK(p != nullptr, HipError, "grad_sqnorm_multi_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    return static_cast<double*>(g_scratch_ptr[dev]);
}

}  // namespace

void grad_sqnorm_multi_noalloc(const float* const* grads, const int64_t* sizes, int count, double* sqnorm,
                               int* nonfinite, hipStream_t s) {
    AIC_CHECK(count >= 0 && sqnorm && nonfinite, InvalidArgument, "grad_sqnorm_multi_noalloc: bad arguments");
    AIC_CHECK(count <= kMaxNormTensors, InvalidArgument, "grad_sqnorm_multi_noalloc: at most ", kMaxNormTensors,
              " tensors");
    int blocks[kMaxNormTensors];
    const int64_t total = sqnorm_blocks(sizes, count, blocks);
    AIC_CHECK(total <= kNoAllocMaxBlocks, OutOfRange, "grad_sqnorm_multi_noalloc: the tensors need ", total,
              " partial blocks (min(ceil(n / 4096), 1024) each), above the fixed scratch of ", kNoAllocMaxBlocks);
    double* pd = device_scratch();
    int* pn = reinterpret_cast<int*>(pd + kNoAllocMaxBlocks);
    sqnorm_launch(grads, sizes, count, blocks, static_cast<int>(total), pd, pn, sqnorm, nonfinite, s);
}

int64_t sqnorm_slots(const int64_t* sizes, int count) {
    AIC_CHECK(count >= 0 && count <= kMaxNormTensors, InvalidArgument, "sqnorm_slots: 0 to ", kMaxNormTensors,
              " tensors");
    int blocks[kMaxNormTensors];
    return sqnorm_blocks(sizes, count, blocks);
}

void sqnorm_partials(const float* const* grads, const int64_t* sizes, int count, double* pd, int* pn,
                     hipStream_t s) {
    AIC_CHECK(count >= 0 && count <= kMaxNormTensors && pd && pn, InvalidArgument, "sqnorm_partials: bad arguments");
    int blocks[kMaxNormTensors];
    sqnorm_blocks(sizes, count, blocks);
    // kSqMultiMax tensors per launch
    int64_t off = 0;
    for (int t0 = 0; t0 < count; t0 += kSqMultiMax) {
        SqMulti m;
        m.count = std::min(count - t0, kSqMultiMax);
        m.first[0] = 0;
        for (int i = 0; i < m.count; ++i) {
            m.g[i] = grads[t0 + i];
            m.n[i] = sizes[t0 + i];
            m.first[i + 1] = m.first[i] + blocks[t0 + i];
        }
        hipLaunchKernelGGL(sqnorm_multi_k, dim3(m.first[m.count]), dim3(256), 0, s, m, pd + off, pn + off);
        AIC_LAUNCH_CHECK("grad_sqnorm_multi");
        off += m.first[m.count];
    }
}

void sqnorm_clear(double* pd, int* pn, int64_t nslots, hipStream_t s) {
    if (nslots <= 0) return;
    hipLaunchKernelGGL(sqslot_clear_k, dim3(static_cast<unsigned>(std::min<int64_t>((nslots + 255) / 256, 1024))),
                       dim3(256), 0, s, pd, pn, nslots);
    AIC_LAUNCH_CHECK("sqslot_clear");
}

int64_t sqnorm_reduce_tmp(int64_t nslots) { return std::max<int64_t>(1, (nslots + 4095) / 4096); }

void sqnorm_reduce(const double* pd, const int* pn, int64_t nslots, double* tmp_d, int* tmp_n, double* sqnorm,
                   int* nonfinite, hipStream_t s) {
    AIC_CHECK(nslots >= 0 && pd && pn && tmp_d && tmp_n && sqnorm && nonfinite, InvalidArgument,
              "sqnorm_reduce: bad arguments");
    const int64_t nb = sqnorm_reduce_tmp(nslots);
    AIC_CHECK(nb <= (int64_t{1} << 20), InvalidArgument, "sqnorm_reduce: too many slots");
    hipLaunchKernelGGL(sqsum_level1_k, dim3(static_cast<unsigned>(nb)), dim3(1024), 0, s, pd, pn, nslots, tmp_d, tmp_n);
    AIC_LAUNCH_CHECK("sqsum_level1");
    hipLaunchKernelGGL(sqnorm_final_k, dim3(1), dim3(1024), 0, s, tmp_d, tmp_n, static_cast<int>(nb), sqnorm,
                       nonfinite);
    AIC_LAUNCH_CHECK("grad_sqnorm_final");
}

void scale_multi(float* const* grads, const int64_t* sizes, int count, const float* scale, hipStream_t s) {
    for (int t = 0; t < count; ++t) {
        if (sizes[t] == 0) continue;
        hipLaunchKernelGGL(scale_k, dim3(grid_for(sizes[t], 256, 8192)), dim3(256), 0, s, grads[t], sizes[t], scale);
        AIC_LAUNCH_CHECK("scale_multi");
    }
}

void optim_finalize(const double* sqnorm, const int* nonfinite, void* ctl, hipStream_t s) {
    AIC_CHECK(sqnorm && nonfinite && ctl, InvalidArgument, "optim_finalize: null argument");
    hipLaunchKernelGGL(finalize_k, dim3(1), dim3(1), 0, s, sqnorm, nonfinite, static_cast<aic_optim_ctl*>(ctl));
    AIC_LAUNCH_CHECK("optim_finalize");
}

void adamw_multi(float* const* p, const float* const* g, float* const* m, float* const* v, void* const* p_bf16,
                 const int64_t* sizes, int count, float lr, float beta1, float beta2, float eps, float wd,
                 int64_t step, const void* ctl, hipStream_t s) {
    AIC_CHECK(ctl || step > 0, InvalidArgument, "adamw_multi: step must be >= 1 without a control block");
    for (int t = 0; t < count; ++t) {
        if (sizes[t] == 0) continue;
        const unsigned grid = grid_for((sizes[t] + 7) / 8, 256, 262144);
        const auto* c = static_cast<const aic_optim_ctl*>(ctl);
        bf16* pb = p_bf16 ? static_cast<bf16*>(p_bf16[t]) : nullptr;
        if (pb)
            hipLaunchKernelGGL(adamw_k<true>, dim3(grid), dim3(256), 0, s, p[t], g[t], m[t], v[t], pb, sizes[t], lr,
                               beta1, beta2, eps, wd, step, 0.0f, 0.0f, c);
        else
            hipLaunchKernelGGL(adamw_k<false>, dim3(grid), dim3(256), 0, s, p[t], g[t], m[t], v[t], pb, sizes[t], lr,
                               beta1, beta2, eps, wd, step, 0.0f, 0.0f, c);
        AIC_LAUNCH_CHECK("adamw");
    }
}

void adamw_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2, float eps,
                float wd, float bc1, float bc2, hipStream_t s) {
    AIC_CHECK(n >= 0 && (n == 0 || (p && g && m && v)), InvalidArgument, "adamw_step: bad arguments");
    AIC_CHECK(bc1 > 0.0f && bc2 > 0.0f, InvalidArgument, "adamw_step: bias corrections must be positive");
    if (n == 0) return;
    const unsigned grid = grid_for((n + 7) / 8, 256, 262144);
    hipLaunchKernelGGL(adamw_k<false>, dim3(grid), dim3(256), 0, s, p, g, m, v, nullptr, n, lr, beta1, beta2, eps, wd,
                       int64_t{0}, bc1, bc2, nullptr);
    AIC_LAUNCH_CHECK("adamw_step");
}

void cast_f32_bf16(const float* src, void* dst, int64_t n, hipStream_t s) {
    if (n == 0) return;
    hipLaunchKernelGGL(cast_k, dim3(grid_for(n, 256, 16384)), dim3(256), 0, s, src, static_cast<bf16*>(dst), n);
    AIC_LAUNCH_CHECK("cast_f32_bf16");
}

void fill_normal(float* dst, int64_t n, uint64_t seed, uint64_t offset, float mean, float std, hipStream_t s) {
    if (n == 0) return;
    hipLaunchKernelGGL(fill_normal_k, dim3(grid_for(n, 256, 16384)), dim3(256), 0, s, dst, n, seed, offset, mean, std);
    AIC_LAUNCH_CHECK("fill_normal");
}

void fill_const(float* dst, int64_t n, float v, hipStream_t s) {
    if (n == 0) return;
    hipLaunchKernelGGL(fill_const_k, dim3(grid_for(n, 256, 16384)), dim3(256), 0, s, dst, n, v);
    AIC_LAUNCH_CHECK("fill_const");
}

namespace {
// one thread: appends the step's statistics to the ring (slot = count % cap) and advances count
__global__ void step_record_k(const float* loss, const float* aux, const aic_optim_ctl* ctl, const float* scale_used,
                              aic_step_record* ring, int64_t* count, int cap) {
    const int64_t i = *count;
    aic_step_record r;
    r.step = ctl->step;
    r.loss = *loss;
    r.aux_loss = aux ? *aux : 0.0f;
    r.grad_norm = ctl->grad_norm;
    r.loss_scale = *scale_used;
    r.found_inf = ctl->skip;
    r.pad = 0;
    ring[i % cap] = r;
    *count = i + 1;
}
}  // namespace

void step_record(const float* loss, const float* aux, const void* ctl, const float* scale_used, void* ring,
                 int64_t* count, int cap, hipStream_t s) {
    AIC_CHECK(loss && ctl && scale_used && ring && count && cap > 0, InvalidArgument, "step_record: bad arguments");
    hipLaunchKernelGGL(step_record_k, dim3(1), dim3(1), 0, s, loss, aux, static_cast<const aic_optim_ctl*>(ctl),
                       scale_used, static_cast<aic_step_record*>(ring), count, cap);
    AIC_LAUNCH_CHECK("step_record");
}

}  // namespace aic::hip
