// Fused log-sum-exp cross-entropy with index or soft targets.
// Replaces cuda_cross_entropy_forward/backward (src/cuda/cuda_loss.cu:68-190) and the CPU
// path of src/loss/cross_entropy.cpp:149-290.  One block per row; the mean over valid rows
// is reduced by a single block in a fixed order (deterministic), and the valid-row count
// stays on the device (the reference synchronises the host for it, cuda_loss.cu:228-234).
// An index target outside [0, C) that is not ignore_index counts as a valid row with loss
// lse - 0 and gradient softmax (no one-hot), as the CUDA launcher computes it
// (cuda_loss.cu:114-121, 170-176; the CPU path throws OutOfRange on the host instead).
// Soft targets y [N, C] (fp32): row loss lse - sum_j y_j z_j, gradient (softmax - y) * scale,
// every row valid (cuda_loss.cu:123-131, 177-184).
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

template <bool PRECISE>
__device__ __forceinline__ float ex(float x) {
    if constexpr (PRECISE) return expf(x);
    else return __expf(x);
}

template <typename T, bool PRECISE>
__global__ __launch_bounds__(256) void ce_fwd_k(const T* __restrict__ logits, int64_t ldl,
                                                const int64_t* __restrict__ targets, int C, int64_t ignore_index,
                                                float* __restrict__ losses, float* __restrict__ lse_out) {
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    const T* z = logits + row * ldl;
    float m = -INFINITY, s = 0.0f;
    for (int j = threadIdx.x; j < C; j += 256) {
        const float v = ld(z, j);
        if (v > m) {
            s = s * ex<PRECISE>(m - v) + 1.0f;
            m = v;
        } else {
            s += ex<PRECISE>(v - m);
        }
    }
    const float M = block_max(m, red);
    const float part = (m == -INFINITY) ? 0.0f : s * ex<PRECISE>(m - M);
    const float S = block_sum(part, red);
    if (threadIdx.x == 0) {
        const float lse = M + logf(fmaxf(S, 1e-12f));
        if (lse_out) lse_out[row] = lse;
        const int64_t t = targets[row];
        float li = 0.0f;
        if (t != ignore_index) li = lse - ((t >= 0 && t < C) ? ld(z, t) : 0.0f);
        if (losses) losses[row] = li;
    }
}

// Single block: recomputes the row losses' sum in a fixed order from `losses`.
__global__ __launch_bounds__(1024) void ce_mean_k(const float* __restrict__ losses,
                                                  const int64_t* __restrict__ targets, int64_t N,
                                                  int64_t ignore_index, float* loss_mean, int64_t* valid) {
    __shared__ double sd[1024];
    __shared__ long long sc[1024];
    double acc = 0.0;
    long long cnt = 0;
    for (int64_t i = threadIdx.x; i < N; i += 1024) {
        acc += static_cast<double>(losses[i]);
        cnt += (!targets || targets[i] != ignore_index) ? 1 : 0;  // no targets: every row (soft targets)
    }
    sd[threadIdx.x] = acc;
    sc[threadIdx.x] = cnt;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            sd[threadIdx.x] += sd[threadIdx.x + o];
            sc[threadIdx.x] += sc[threadIdx.x + o];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const long long v = sc[0];
        if (valid) *valid = v;
        if (loss_mean) *loss_mean = v > 0 ? static_cast<float>(sd[0]) / static_cast<float>(v) : 0.0f;
    }
}

// Row weight of the gradient, as CrossEntropyBackward scales it (src/loss/cross_entropy.cpp:86-105):
// per_row ("none"): grad[row] (1 without grad); otherwise grad[0] (1 without grad) divided by the
// valid-row count -- *valid from the device when given, else the host's divisor ("mean": the
// count, "sum": 1) -- and 0 when that count is 0.
struct RowWeight {
    const float* grad;
    const int64_t* valid;
    float divisor;
    int per_row;
    __device__ __forceinline__ float operator()(int64_t row) const {
        if (per_row) return grad ? grad[row] : 1.0f;
        const float g = grad ? *grad : 1.0f;
        const float dv = valid ? static_cast<float>(*valid) : divisor;
        return dv > 0.0f ? g / dv : 0.0f;
    }
};

template <typename T, bool PRECISE>
__global__ __launch_bounds__(256) void ce_bwd_k(const T* logits, int64_t ldl, const int64_t* __restrict__ targets,
                                                const float* __restrict__ lse, int C, int64_t ignore_index,
                                                RowWeight rw, T* dl, int64_t ldd) {
    const int64_t row = blockIdx.x;
    const int64_t t = targets[row];
    const T* z = logits + row * ldl;
    T* d = dl + row * ldd;
    if (t == ignore_index) {
        for (int j = threadIdx.x; j < C; j += 256) st(d, j, 0.0f);
        return;
    }
    const float scale = rw(row);
    const float l = lse[row];
    for (int j = threadIdx.x; j < C; j += 256) {
        const float p = ex<PRECISE>(ld(z, j) - l);
        st(d, j, (p - (j == t ? 1.0f : 0.0f)) * scale);
    }
}

// bf16 rows with C % 8 == 0 and 16-byte aligned rows: 8 logits per access.
__global__ __launch_bounds__(256) void ce_fwd_bf16v(const bf16* __restrict__ logits, int64_t ldl,
                                                    const int64_t* __restrict__ targets, int C,
                                                    int64_t ignore_index, float* __restrict__ losses,
                                                    float* __restrict__ lse_out) {
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    const bf16* z = logits + row * ldl;
    float m = -INFINITY, s = 0.0f;
    for (int j = threadIdx.x * 8; j < C; j += 256 * 8) {
        const uint4 raw = *reinterpret_cast<const uint4*>(z + j);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
        float mx = v[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mx = fmaxf(mx, v[i]);
        if (mx > m) {
            s *= __expf(m - mx);
            m = mx;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) s += __expf(v[i] - m);
    }
    const float M = block_max(m, red);
    const float part = (m == -INFINITY) ? 0.0f : s * __expf(m - M);
    const float S = block_sum(part, red);
    if (threadIdx.x == 0) {
        const float lse = M + logf(fmaxf(S, 1e-12f));
        if (lse_out) lse_out[row] = lse;
        const int64_t t = targets[row];
        float li = 0.0f;
        if (t != ignore_index) li = lse - ((t >= 0 && t < C) ? bf2f(z[t]) : 0.0f);
        if (losses) losses[row] = li;
    }
}

__global__ __launch_bounds__(256) void ce_bwd_bf16v(const bf16* logits, int64_t ldl,
                                                    const int64_t* __restrict__ targets, const float* __restrict__ lse,
                                                    int C, int64_t ignore_index, RowWeight rw, bf16* dl, int64_t ldd) {
    const int64_t row = blockIdx.x;
    const int64_t t = targets[row];
    const bf16* z = logits + row * ldl;
    bf16* d = dl + row * ldd;
    const bool ign = (t == ignore_index);
    const float scale = ign ? 0.0f : rw(row);
    const float l = ign ? 0.0f : lse[row];
    for (int j = threadIdx.x * 8; j < C; j += 256 * 8) {
        const uint4 raw = *reinterpret_cast<const uint4*>(z + j);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = __uint_as_float(w[i] << 16), b = __uint_as_float(w[i] & 0xffff0000u);
            float ga = (__expf(a - l) - (j + 2 * i == t ? 1.0f : 0.0f)) * scale;
            float gb = (__expf(b - l) - (j + 2 * i + 1 == t ? 1.0f : 0.0f)) * scale;
            if (ign) ga = gb = 0.0f;
            o[i] = pack_bf16x2(ga, gb);
        }
        *reinterpret_cast<uint4*>(d + j) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Rows with a target other than ignore_index (single block, fixed order).
__global__ __launch_bounds__(1024) void ce_count_k(const int64_t* __restrict__ targets, int64_t N,
                                                   int64_t ignore_index, int64_t* valid) {
    __shared__ long long sc[1024];
    long long cnt = 0;
    for (int64_t i = threadIdx.x; i < N; i += 1024) cnt += (targets[i] != ignore_index) ? 1 : 0;
    sc[threadIdx.x] = cnt;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if (threadIdx.x < o) sc[threadIdx.x] += sc[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) *valid = sc[0];
}

// Forward and backward of one bf16 row in one pass (C % 8 == 0, C <= 2048 NIT): the row is read
// once into registers (NIT 16-byte chunks per thread, in ce_fwd_bf16v's order, so the LSE and
// the row loss are that kernel's), then overwritten by ce_bwd_bf16v's gradient.  The target
// logit is read before the barrier that precedes every write.
template <int NIT>
__global__ __launch_bounds__(256) void ce_fused_bf16v(bf16* logits, int64_t ldl, const int64_t* __restrict__ targets,
                                                      int C, int64_t ignore_index, float* __restrict__ losses,
                                                      float* __restrict__ lse_out, RowWeight rw) {
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    bf16* z = logits + row * ldl;
    const int64_t t = targets[row];
    const bool ign = t == ignore_index, tin = t >= 0 && t < C;
    float zt = 0.0f;
    if (threadIdx.x == 0 && !ign && tin) zt = bf2f(z[t]);
    uint4 raw[NIT];
    float m = -INFINITY, s = 0.0f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int j = (it * 256 + threadIdx.x) * 8;
        raw[it] = j < C ? *reinterpret_cast<const uint4*>(z + j) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int j = (it * 256 + threadIdx.x) * 8;
        if (j >= C) continue;
        const uint32_t w[4] = {raw[it].x, raw[it].y, raw[it].z, raw[it].w};
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
        float mx = v[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mx = fmaxf(mx, v[i]);
        if (mx > m) {
            s *= __expf(m - mx);
            m = mx;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) s += __expf(v[i] - m);
    }
    const float M = block_max(m, red);
    const float part = (m == -INFINITY) ? 0.0f : s * __expf(m - M);
    const float S = block_sum(part, red);
    const float lse = M + logf(fmaxf(S, 1e-12f));
    if (threadIdx.x == 0) {
        if (lse_out) lse_out[row] = lse;
        if (losses) losses[row] = ign ? 0.0f : lse - (tin ? zt : 0.0f);
    }
    const float scale = ign ? 0.0f : rw(row);
    const float l = ign ? 0.0f : lse;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int j = (it * 256 + threadIdx.x) * 8;
        if (j >= C) continue;
        const uint32_t w[4] = {raw[it].x, raw[it].y, raw[it].z, raw[it].w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = __uint_as_float(w[i] << 16), b = __uint_as_float(w[i] & 0xffff0000u);
            float ga = (__expf(a - l) - (j + 2 * i == t ? 1.0f : 0.0f)) * scale;
            float gb = (__expf(b - l) - (j + 2 * i + 1 == t ? 1.0f : 0.0f)) * scale;
            if (ign) ga = gb = 0.0f;
            o[i] = pack_bf16x2(ga, gb);
        }
        *reinterpret_cast<uint4*>(z + j) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Soft targets: the row's online log-sum-exp as ce_fwd_k and its dot product with y (block sums).
template <typename T, bool PRECISE>
__global__ __launch_bounds__(256) void ce_soft_fwd_k(const T* __restrict__ logits, int64_t ldl,
                                                     const float* __restrict__ y, int64_t ldy, int C,
                                                     float* __restrict__ losses, float* __restrict__ lse_out) {
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    const T* z = logits + row * ldl;
    const float* yr = y + row * ldy;
    float m = -INFINITY, s = 0.0f, dot = 0.0f;
    for (int j = threadIdx.x; j < C; j += 256) {
        const float v = ld(z, j);
        dot += yr[j] * v;
        if (v > m) {
            s = s * ex<PRECISE>(m - v) + 1.0f;
            m = v;
        } else {
            s += ex<PRECISE>(v - m);
        }
    }
    const float M = block_max(m, red);
    const float part = (m == -INFINITY) ? 0.0f : s * ex<PRECISE>(m - M);
    const float S = block_sum(part, red);
    const float D = block_sum(dot, red);
    if (threadIdx.x == 0) {
        const float lse = M + logf(fmaxf(S, 1e-12f));
        if (lse_out) lse_out[row] = lse;
        if (losses) losses[row] = lse - D;
    }
}

template <typename T, bool PRECISE>
__global__ __launch_bounds__(256) void ce_soft_bwd_k(const T* logits, int64_t ldl, const float* __restrict__ y,
                                                     int64_t ldy, const float* __restrict__ lse, int C, RowWeight rw,
                                                     T* dl, int64_t ldd) {
    const int64_t row = blockIdx.x;
    const T* z = logits + row * ldl;
    const float* yr = y + row * ldy;
    T* d = dl + row * ldd;
    const float scale = rw(row);
    const float l = lse[row];
    for (int j = threadIdx.x; j < C; j += 256) st(d, j, (ex<PRECISE>(ld(z, j) - l) - yr[j]) * scale);
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

void ce_fwd(const void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
            float* losses, float* lse, float* loss_mean, int64_t* valid, DType dt, hipStream_t s) {
    AIC_CHECK(N >= 0 && C > 0 && ld >= C && C < (1LL << 31), InvalidArgument, "ce_fwd: bad shape");
    AIC_CHECK(N < (1LL << 31), InvalidArgument, "ce_fwd: too many rows");
    float* tmp = nullptr;
    DeviceBuffer hold;
    if (N > 0) {
        if (!losses && (loss_mean || valid)) {
            hold = DeviceBuffer(sizeof(float) * N, s);
            tmp = hold.as<float>();
        }
        float* lp = losses ? losses : tmp;
        const dim3 grid(static_cast<unsigned>(N));
        if (dt == DType::BFloat16 && C % 8 == 0 && ld % 8 == 0 && a16(logits))
            hipLaunchKernelGGL(ce_fwd_bf16v, grid, dim3(256), 0, s, static_cast<const bf16*>(logits), ld, targets,
                               static_cast<int>(C), ignore_index, lp, lse);
        else if (dt == DType::BFloat16)
            hipLaunchKernelGGL((ce_fwd_k<bf16, false>), grid, dim3(256), 0, s, static_cast<const bf16*>(logits), ld,
                               targets, static_cast<int>(C), ignore_index, lp, lse);
        else if (dt == DType::Float32)
            hipLaunchKernelGGL((ce_fwd_k<float, true>), grid, dim3(256), 0, s, static_cast<const float*>(logits), ld,
                               targets, static_cast<int>(C), ignore_index, lp, lse);
        else
            AIC_THROW(DTypeMismatch, "ce_fwd: dtype must be f32 or bf16");
        AIC_LAUNCH_CHECK("ce_fwd");
    }
    if (loss_mean || valid) {
        const float* lp = losses ? losses : tmp;
        hipLaunchKernelGGL(ce_mean_k, dim3(1), dim3(1024), 0, s, lp, targets, N, ignore_index, loss_mean, valid);
        AIC_LAUNCH_CHECK("ce_mean");
    }
}

namespace {

void ce_bwd_launch(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                   int64_t ignore_index, RowWeight w, void* dlogits, int64_t ld_d, DType dt, hipStream_t s) {
    AIC_CHECK(N >= 0 && C > 0 && ld >= C && ld_d >= C && C < (1LL << 31), InvalidArgument, "ce_bwd: bad shape");
    AIC_CHECK(lse && targets, InvalidArgument, "ce_bwd: targets and lse are required");
    if (N == 0) return;
    const dim3 grid(static_cast<unsigned>(N));
    if (dt == DType::BFloat16 && C % 8 == 0 && ld % 8 == 0 && ld_d % 8 == 0 && a16(logits) && a16(dlogits))
        hipLaunchKernelGGL(ce_bwd_bf16v, grid, dim3(256), 0, s, static_cast<const bf16*>(logits), ld, targets, lse,
                           static_cast<int>(C), ignore_index, w, static_cast<bf16*>(dlogits), ld_d);
    else if (dt == DType::BFloat16)
        hipLaunchKernelGGL((ce_bwd_k<bf16, false>), grid, dim3(256), 0, s, static_cast<const bf16*>(logits), ld,
                           targets, lse, static_cast<int>(C), ignore_index, w, static_cast<bf16*>(dlogits), ld_d);
    else if (dt == DType::Float32)
        hipLaunchKernelGGL((ce_bwd_k<float, true>), grid, dim3(256), 0, s, static_cast<const float*>(logits), ld,
                           targets, lse, static_cast<int>(C), ignore_index, w, static_cast<float*>(dlogits), ld_d);
    else
        AIC_THROW(DTypeMismatch, "ce_bwd: dtype must be f32 or bf16");
    AIC_LAUNCH_CHECK("ce_bwd");
}

}  // namespace

void ce_bwd(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N, int64_t C,
            int64_t ignore_index, const float* grad, const int64_t* valid, void* dlogits, int64_t ld_d, DType dt,
            hipStream_t s) {
    AIC_CHECK(grad && valid, InvalidArgument, "ce_bwd: grad and valid are required");
    ce_bwd_launch(logits, ld, targets, lse, N, C, ignore_index, RowWeight{grad, valid, 0.0f, 0}, dlogits, ld_d, dt,
                  s);
}

void ce_bwd_rows(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                 int64_t ignore_index, const float* grad, int per_row, float divisor, void* dlogits, int64_t ld_d,
                 DType dt, hipStream_t s) {
    AIC_CHECK(per_row || divisor >= 0.0f, InvalidArgument, "ce_bwd_rows: negative divisor");
    ce_bwd_launch(logits, ld, targets, lse, N, C, ignore_index, RowWeight{grad, nullptr, divisor, per_row ? 1 : 0},
                  dlogits, ld_d, dt, s);
}

void ce_fwd_soft(const void* logits, int64_t ld, const float* y, int64_t ldy, int64_t N, int64_t C, float* losses,
                 float* lse, float* loss_mean, DType dt, hipStream_t s) {
    AIC_CHECK(N >= 0 && C > 0 && ld >= C && ldy >= C && C < (1LL << 31) && N < (1LL << 31), InvalidArgument,
              "ce_fwd_soft: bad shape");
    AIC_CHECK(y || N == 0, InvalidArgument, "ce_fwd_soft: targets are required");
    DeviceBuffer hold;
    float* lp = losses;
    if (N > 0 && !lp && loss_mean) {
        hold = DeviceBuffer(sizeof(float) * N, s);
        lp = hold.as<float>();
    }
    if (N > 0) {
        const dim3 grid(static_cast<unsigned>(N));
        if (dt == DType::Float32)
            hipLaunchKernelGGL((ce_soft_fwd_k<float, true>), grid, dim3(256), 0, s, static_cast<const float*>(logits),
                               ld, y, ldy, static_cast<int>(C), lp, lse);
        else if (dt == DType::BFloat16)
            hipLaunchKernelGGL((ce_soft_fwd_k<bf16, false>), grid, dim3(256), 0, s, static_cast<const bf16*>(logits),
                               ld, y, ldy, static_cast<int>(C), lp, lse);
        else
            AIC_THROW(DTypeMismatch, "ce_fwd_soft: dtype must be f32 or bf16");
        AIC_LAUNCH_CHECK("ce_soft_fwd");
    }
    if (loss_mean) {
        hipLaunchKernelGGL(ce_mean_k, dim3(1), dim3(1024), 0, s, lp, nullptr, N, int64_t{0}, loss_mean, nullptr);
        AIC_LAUNCH_CHECK("ce_mean");
    }
}

void ce_bwd_soft(const void* logits, int64_t ld, const float* y, int64_t ldy, const float* lse, int64_t N, int64_t C,
                 const float* grad, int per_row, float divisor, void* dlogits, int64_t ld_d, DType dt, hipStream_t s) {
    AIC_CHECK(N >= 0 && C > 0 && ld >= C && ldy >= C && ld_d >= C && C < (1LL << 31) && N < (1LL << 31),
              InvalidArgument, "ce_bwd_soft: bad shape");
    AIC_CHECK((y && lse) || N == 0, InvalidArgument, "ce_bwd_soft: targets and lse are required");
    AIC_CHECK(per_row || divisor >= 0.0f, InvalidArgument, "ce_bwd_soft: negative divisor");
    if (N == 0) return;
    const RowWeight w{grad, nullptr, divisor, per_row ? 1 : 0};
    const dim3 grid(static_cast<unsigned>(N));
    if (dt == DType::Float32)
        hipLaunchKernelGGL((ce_soft_bwd_k<float, true>), grid, dim3(256), 0, s, static_cast<const float*>(logits), ld,
                           y, ldy, lse, static_cast<int>(C), w, static_cast<float*>(dlogits), ld_d);
    else if (dt == DType::BFloat16)
        hipLaunchKernelGGL((ce_soft_bwd_k<bf16, false>), grid, dim3(256), 0, s, static_cast<const bf16*>(logits), ld,
                           y, ldy, lse, static_cast<int>(C), w, static_cast<bf16*>(dlogits), ld_d);
    else
        AIC_THROW(DTypeMismatch, "ce_bwd_soft: dtype must be f32 or bf16");
    AIC_LAUNCH_CHECK("ce_soft_bwd");
}

}  // namespace aic::hip

namespace aic::hip {

void ce_fwd_bwd(void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
                float* losses, float* lse, float* loss_mean, int64_t* valid, const float* grad, DType dt,
                hipStream_t s) {
    AIC_CHECK(N >= 0 && C > 0 && ld >= C && C < (1LL << 31) && N < (1LL << 31), InvalidArgument,
              "ce_fwd_bwd: bad shape");
    AIC_CHECK(valid && (targets || N == 0), InvalidArgument, "ce_fwd_bwd: targets and valid are required");
    if (N == 0) {
        ce_fwd(logits, ld, targets, N, C, ignore_index, losses, lse, loss_mean, valid, dt, s);
        return;
    }
    DeviceBuffer hold_l, hold_s;
    float* lp = losses;
    float* sp = lse;
    if (!lp) {
        hold_l = DeviceBuffer(sizeof(float) * N, s);
        lp = hold_l.as<float>();
    }
    if (!sp) {
        hold_s = DeviceBuffer(sizeof(float) * N, s);
        sp = hold_s.as<float>();
    }
    hipLaunchKernelGGL(ce_count_k, dim3(1), dim3(1024), 0, s, targets, N, ignore_index, valid);
    AIC_LAUNCH_CHECK("ce_count");
    const int64_t nit = (C + 2047) / 2048;
    if (dt == DType::BFloat16 && C % 8 == 0 && ld % 8 == 0 && a16(logits) && nit <= 32) {
        const RowWeight rw{grad, valid, 0.0f, 0};
        const dim3 grid(static_cast<unsigned>(N));
        bf16* z = static_cast<bf16*>(logits);
        const int c = static_cast<int>(C);
#define AIC_CE_FUSED(NIT) \
    hipLaunchKernelGGL(ce_fused_bf16v<NIT>, grid, dim3(256), 0, s, z, ld, targets, c, ignore_index, lp, sp, rw)
        if (nit <= 1) AIC_CE_FUSED(1);
        else if (nit <= 2) AIC_CE_FUSED(2);
        else if (nit <= 4) AIC_CE_FUSED(4);
        else if (nit <= 8) AIC_CE_FUSED(8);
        else if (nit <= 16) AIC_CE_FUSED(16);
        else AIC_CE_FUSED(32);
#undef AIC_CE_FUSED
        AIC_LAUNCH_CHECK("ce_fused");
    } else {
        // two passes with the same results: the row losses and LSE, then the gradient in place
        ce_fwd(logits, ld, targets, N, C, ignore_index, lp, sp, nullptr, nullptr, dt, s);
        ce_bwd_launch(logits, ld, targets, sp, N, C, ignore_index, RowWeight{grad, valid, 0.0f, 0}, logits, ld, dt, s);
    }
    if (loss_mean) {
        hipLaunchKernelGGL(ce_mean_k, dim3(1), dim3(1024), 0, s, lp, targets, N, ignore_index, loss_mean, valid);
        AIC_LAUNCH_CHECK("ce_mean");
    }
}

}  // namespace aic::hip
