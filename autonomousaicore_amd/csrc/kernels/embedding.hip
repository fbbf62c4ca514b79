// Token embedding gather and its deterministic scatter-add backward.
// Replaces cuda_embedding_forward/backward (src/cuda/cuda_embedding.cu:21-61), whose
// backward uses fp32 atomicAdd (order-dependent results).  Here the backward sorts the
// (id, position) pairs (chunks of 2048 sorted in LDS by as many blocks, then merged by rank:
// each key's place is its index in its chunk plus its lower bound in every other chunk) and
// sums each id's rows in a fixed order (interleaved chains over the token-ordered run, then
// the chains in order), so repeated runs are bit-identical and ids that repeat often
// (Zipf-distributed text) are summed by sixteen waves instead of serialising on one address;
// runs of at most sixteen ids are summed by one wave each, in token order.
// Rows of ids that do not occur are written as zeros by their own kernel (no separate clear of
// the whole gradient, and no memset node for a captured graph).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void embed_fwd_k(const int64_t* __restrict__ ids, int64_t N, const T* __restrict__ W,
                                                   int64_t V, int64_t D, T* __restrict__ out) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= N * D) return;
    const int64_t i = idx / D, d = idx % D;
    const int64_t t = ids[i];
    out[idx] = (t >= 0 && t < V) ? W[t * D + d] : T(0.0f);
}

// 16-byte copies (D*sizeof(T) % 16 == 0).
__global__ __launch_bounds__(256) void embed_fwd_v(const int64_t* __restrict__ ids, int64_t N,
                                                   const uint4* __restrict__ W, int64_t V, int64_t Dv,
                                                   uint4* __restrict__ out) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= N * Dv) return;
    const int64_t i = idx / Dv, d = idx % Dv;
    const int64_t t = ids[i];
    out[idx] = (t >= 0 && t < V) ? W[t * Dv + d] : make_uint4(0, 0, 0, 0);
}

constexpr int kSortChunk = 2048;          // keys sorted per block in LDS (16 KB)
constexpr int64_t kMaxTokens = 1LL << 20;  // tokens per call (the merge costs log2(2048) probes per other chunk)

// Key of token i: id << 32 | i; ids outside [0, V) sort last (as 0x7fffffff).
__device__ __forceinline__ unsigned long long embed_key(const int64_t* __restrict__ ids, int i, int64_t V) {
    const int64_t t = ids[i];
    const unsigned long long id = (t >= 0 && t < V) ? static_cast<unsigned long long>(t) : 0x7fffffffull;
    return (id << 32) | static_cast<unsigned long long>(i);
}

// Block c sorts the keys of tokens [c * 2048, (c + 1) * 2048) ascending (bitonic in LDS).
__global__ __launch_bounds__(1024) void embed_chunk_sort_k(const int64_t* __restrict__ ids, int N, int64_t V,
                                                           unsigned long long* __restrict__ sk) {
    __shared__ unsigned long long key[kSortChunk];
    const int c0 = static_cast<int>(blockIdx.x) * kSortChunk, n = min(kSortChunk, N - c0);
    for (int i = threadIdx.x; i < kSortChunk; i += blockDim.x) key[i] = i < n ? embed_key(ids, c0 + i, V) : ~0ull;
    __syncthreads();
    for (int size = 2; size <= kSortChunk; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < kSortChunk; i += blockDim.x) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;
                    const unsigned long long a = key[i], b = key[j];
                    if ((a > b) == up) {
                        key[i] = b;
                        key[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < n; i += blockDim.x) sk[c0 + i] = key[i];
}

// The merged order: key g of chunk c lands at its index within c plus, for every other chunk,
// the number of that chunk's keys below it (keys are unique, so this is a permutation).
__global__ __launch_bounds__(256) void embed_merge_rank_k(const unsigned long long* __restrict__ sk, int N,
                                                          int* __restrict__ sorted_pos, int* __restrict__ sorted_id) {
    const int g = static_cast<int>(blockIdx.x) * 256 + threadIdx.x;
    if (g >= N) return;
    const unsigned long long k = sk[g];
    const int c = g / kSortChunk, nchunks = (N + kSortChunk - 1) / kSortChunk;
    int rank = g - c * kSortChunk;
    for (int o = 0; o < nchunks; ++o) {
        if (o == c) continue;
        const unsigned long long* base = sk + static_cast<int64_t>(o) * kSortChunk;
        int lo = 0, hi = min(kSortChunk, N - o * kSortChunk);  // lower bound of k in [lo, hi)
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (base[mid] < k) lo = mid + 1;
            else hi = mid;
        }
        rank += lo;
    }
    sorted_pos[rank] = static_cast<int>(k & 0xffffffffull);
    sorted_id[rank] = static_cast<int>(k >> 32);
}

// Runs of at most this many equal ids are summed by one wave in token order; longer ones by a
// block of sixteen waves.
constexpr int kShortRun = 16;

// Starts of the runs of equal in-range ids in the sorted order, compacted, with run_start[nruns]
// = the number of in-range ids (the end of the last run), and the indices of the runs longer than
// kShortRun in long_runs: thread t owns sorted positions [t * per, (t + 1) * per); exclusive scans
// of the per-thread counts give the offsets.  counts[0] = nruns, counts[1] = the long runs.
__global__ __launch_bounds__(1024) void embed_runs_k(const int* __restrict__ sorted_id, int N, int64_t V,
                                                     int* __restrict__ run_start, int* __restrict__ long_runs,
                                                     int* __restrict__ counts) {
    __shared__ int cnt[1024], lcnt[1024];
    const int per = (N + blockDim.x - 1) / blockDim.x;
    const int b0 = threadIdx.x * per, b1 = min(N, b0 + per);
    auto is_start = [&](int i) {
        const int id = sorted_id[i];
        return id < V && (i == 0 || sorted_id[i - 1] != id);
    };
    // sorted, so a run starting at i is longer than kShortRun iff position i + kShortRun holds its id
    auto is_long = [&](int i) { return i + kShortRun < N && sorted_id[i + kShortRun] == sorted_id[i]; };
    int c = 0, l = 0, in_range = 0;
    for (int i = b0; i < b1; ++i) {
        const bool st = is_start(i);
        c += st;
        l += st && is_long(i);
        in_range += sorted_id[i] < V;
    }
    cnt[threadIdx.x] = c;
    lcnt[threadIdx.x] = l;
    __syncthreads();
    for (int off = 1; off < static_cast<int>(blockDim.x); off <<= 1) {  // inclusive Hillis-Steele scans
        const bool has = threadIdx.x >= static_cast<unsigned>(off);
        const int v = has ? cnt[threadIdx.x - off] : 0, w = has ? lcnt[threadIdx.x - off] : 0;
        __syncthreads();
        cnt[threadIdx.x] += v;
        lcnt[threadIdx.x] += w;
        __syncthreads();
    }
    int o = cnt[threadIdx.x] - c, ol = lcnt[threadIdx.x] - l;
    for (int i = b0; i < b1; ++i)
        if (is_start(i)) {
            if (is_long(i)) long_runs[ol++] = o;
            run_start[o++] = i;
        }
    // the in-range ids sort first: the thread holding the last in-range id (or the first
    // thread when none is) writes the end of the last run
    if (in_range > 0 && (b1 == N || sorted_id[b1] >= V)) run_start[cnt[blockDim.x - 1]] = b0 + in_range;
    if (threadIdx.x == 0 && sorted_id[0] >= V) run_start[0] = 0;
    if (threadIdx.x == blockDim.x - 1) {
        counts[0] = cnt[threadIdx.x];
        counts[1] = lcnt[threadIdx.x];
    }
}

// Zeros for the rows of ids that occur nowhere in the sorted ids (one wave per row; a lower
// bound over the sorted ids decides), 16-byte stores when the rows allow them.
__global__ __launch_bounds__(256) void embed_zero_absent_k(const int* __restrict__ sorted_id, int N, int64_t V,
                                                           float* __restrict__ dW, int64_t D, int vec) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= V) return;
    const int lane = threadIdx.x & 63;
    int lo = 0, hi = N;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sorted_id[mid] < row) lo = mid + 1;
        else hi = mid;
    }
    if (lo < N && sorted_id[lo] == row) return;
    float* r = dW + row * D;
    if (vec) {
        for (int64_t c = 4 * lane; c < D; c += 256)
            *reinterpret_cast<float4*>(r + c) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else {
        for (int64_t c = lane; c < D; c += 64) r[c] = 0.0f;
    }
}

// LB bytes of a dout row per lane: the row words of LB / 4 32-bit loads.
template <int LB>
struct RowLoad {
    uint32_t w[LB / 4];
};

template <typename T, int LB>
__device__ __forceinline__ RowLoad<LB> load_row(const T* __restrict__ p) {
    RowLoad<LB> r;
    if constexpr (LB == 16) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        r.w[0] = v.x, r.w[1] = v.y, r.w[2] = v.z, r.w[3] = v.w;
    } else if constexpr (LB == 8) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        r.w[0] = v.x, r.w[1] = v.y;
    } else {
        r.w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
    return r;
}

template <typename T, int LB>
__device__ __forceinline__ void add_row(float* acc, const RowLoad<LB>& r) {
#pragma unroll
    for (int k = 0; k < LB / 4; ++k) {
        if constexpr (sizeof(T) == 2) {
            acc[2 * k] += __uint_as_float(r.w[k] << 16);
            acc[2 * k + 1] += __uint_as_float(r.w[k] & 0xffff0000u);
        } else {
            acc[k] += __uint_as_float(r.w[k]);
        }
    }
}

// Sum of the rows of tokens q0, q0 + step, ... below end, in that order, onto acc: U rows'
// loads in flight at a time.
template <typename T, int LB, int U>
__device__ __forceinline__ void sum_rows(float* acc, const int* __restrict__ sorted_pos, int q0, int end, int step,
                                         const T* __restrict__ dout, int64_t D, int64_t col) {
    for (; q0 < end; q0 += step * U) {
        RowLoad<LB> raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = q0 + step * u;
            if (q < end) raw[u] = load_row<T, LB>(dout + static_cast<int64_t>(sorted_pos[q]) * D + col);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (q0 + step * u >= end) break;
            add_row<T, LB>(acc, raw[u]);
        }
    }
}

// The column sums of every run of equal ids, per chunk of 64 lanes x LB bytes of the row.
// Runs longer than kShortRun first: one block of 16 waves per (long run, chunk), wave w adding
// the rows of tokens p + w, p + w + 16, ... in order, the 16 partial sums then added in wave
// order.  Then the short runs: one wave per (run, chunk), adding the rows in token order.  Both
// orders are fixed by the run length alone, so the result is the same on every run.
template <typename T, int LB>
__global__ __launch_bounds__(1024) void embed_run_k(const int* __restrict__ sorted_pos, const int* __restrict__ sorted_id,
                                                    const int* __restrict__ run_start,
                                                    const int* __restrict__ long_runs, const int* __restrict__ counts,
                                                    const T* __restrict__ dout, int64_t D, float* __restrict__ dW,
                                                    int accumulate) {
    constexpr int VE = LB / sizeof(T);  // elements per lane
    constexpr int CE = 64 * VE;         // columns per chunk
    __shared__ float part[16][CE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunks = static_cast<int>(D / CE);
    const int nruns = counts[0], nlong = counts[1];
    for (int it = blockIdx.x; it < nlong * chunks; it += gridDim.x) {
        const int r = long_runs[it / chunks], ch = it % chunks;
        const int p = run_start[r], end = run_start[r + 1], id = sorted_id[p];
        const int64_t col = static_cast<int64_t>(ch) * CE + lane * VE;
        float acc[VE];
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[e] = 0.0f;
        sum_rows<T, LB, 8>(acc, sorted_pos, p + wave, end, 16, dout, D, col);
#pragma unroll
        for (int e = 0; e < VE; ++e) part[wave][lane * VE + e] = acc[e];
        __syncthreads();
        if (threadIdx.x < CE) {
            float sum = part[0][threadIdx.x];
#pragma unroll
            for (int w = 1; w < 16; ++w) sum += part[w][threadIdx.x];
            float* o = dW + static_cast<int64_t>(id) * D + static_cast<int64_t>(ch) * CE + threadIdx.x;
            *o = accumulate ? *o + sum : sum;
        }
        __syncthreads();
    }
    const int gw = static_cast<int>(blockIdx.x) * 16 + wave, nw = static_cast<int>(gridDim.x) * 16;
    for (int it = gw; it < nruns * chunks; it += nw) {
        const int r = it / chunks, ch = it % chunks;
        const int p = run_start[r], end = run_start[r + 1];
        if (end - p > kShortRun) continue;
        const int id = sorted_id[p];
        const int64_t col = static_cast<int64_t>(ch) * CE + lane * VE;
        float acc[VE];
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[e] = 0.0f;
        sum_rows<T, LB, 8>(acc, sorted_pos, p, end, 1, dout, D, col);
        float* o = dW + static_cast<int64_t>(id) * D + col;
        if constexpr (VE % 4 == 0) {  // 16-byte stores (the caller checks dW's alignment)
#pragma unroll
            for (int e = 0; e < VE; e += 4) {
                float4 v = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
                if (accumulate) {
                    const float4 a = *reinterpret_cast<const float4*>(o + e);
                    v = make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
                }
                *reinterpret_cast<float4*>(o + e) = v;
            }
        } else {
#pragma unroll
            for (int e = 0; e < VE; ++e) o[e] = accumulate ? o[e] + acc[e] : acc[e];
        }
    }
}

// One block per (sorted position p, column chunk of 256).  The block does work only if p
// starts a run of equal ids; its 4 waves take every 4th token of the run, then combine in
// a fixed order.
template <typename T>
__global__ __launch_bounds__(256) void embed_seg_k(const int* __restrict__ sorted_pos, const int* __restrict__ sorted_id,
                                                   int N, int64_t V, const T* __restrict__ dout, int64_t D,
                                                   float* __restrict__ dW, int accumulate) {
    __shared__ float part[4][64];
    const int p = blockIdx.x;
    const int id = sorted_id[p];
    if (id >= V) return;
    if (p > 0 && sorted_id[p - 1] == id) return;
    int end = p + 1;
    while (end < N && sorted_id[end] == id) ++end;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int64_t c0 = static_cast<int64_t>(blockIdx.y) * 64; c0 < D; c0 += static_cast<int64_t>(gridDim.y) * 64) {
        const int64_t c = c0 + lane;
        float acc = 0.0f;
        if (c < D)
            for (int q = p + wave; q < end; q += 4) acc += ld(dout, static_cast<int64_t>(sorted_pos[q]) * D + c);
        part[wave][lane] = acc;
        __syncthreads();
        if (wave == 0 && c < D) {
            const float s = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
            float* o = dW + static_cast<int64_t>(id) * D + c;
            *o = accumulate ? *o + s : s;
        }
        __syncthreads();
    }
}

}  // namespace

void embed_fwd(const int64_t* ids, int64_t N, const void* W, int64_t V, int64_t D, void* out, DType dt, hipStream_t s) {
    AIC_CHECK(N >= 0 && V > 0 && D > 0, InvalidArgument, "embed_fwd: bad shape");
    if (N == 0) return;
    const size_t es = dtype_size(dt);
    AIC_CHECK(dt == DType::Float32 || dt == DType::BFloat16, DTypeMismatch, "embed_fwd: dtype must be f32 or bf16");
    const bool vec = (D * es) % 16 == 0 && (reinterpret_cast<uintptr_t>(W) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
    if (vec) {
        const int64_t Dv = D * static_cast<int64_t>(es) / 16;
        hipLaunchKernelGGL(embed_fwd_v, dim3(grid_for(N * Dv, 256, 1LL << 31)), dim3(256), 0, s, ids, N,
                           static_cast<const uint4*>(W), V, Dv, static_cast<uint4*>(out));
    } else if (dt == DType::Float32) {
        hipLaunchKernelGGL(embed_fwd_k<float>, dim3(grid_for(N * D, 256, 1LL << 31)), dim3(256), 0, s, ids, N,
                           static_cast<const float*>(W), V, D, static_cast<float*>(out));
    } else {
        hipLaunchKernelGGL(embed_fwd_k<bf16>, dim3(grid_for(N * D, 256, 1LL << 31)), dim3(256), 0, s, ids, N,
                           static_cast<const bf16*>(W), V, D, static_cast<bf16*>(out));
    }
    AIC_LAUNCH_CHECK("embed_fwd");
}

void embed_bwd(const int64_t* ids, int64_t N, const void* dout, int64_t V, int64_t D, float* dW, bool accumulate,
               DType dt, hipStream_t s) {
    AIC_CHECK(N >= 0 && V > 0 && D > 0, InvalidArgument, "embed_bwd: bad shape");
    AIC_CHECK(N <= kMaxTokens, InvalidArgument, "embed_bwd: at most ", kMaxTokens, " tokens per call, got ", N);
    AIC_CHECK(V < 0x7fffffffLL, InvalidArgument, "embed_bwd: vocabulary too large");
    AIC_CHECK(dt == DType::Float32 || dt == DType::BFloat16, DTypeMismatch, "embed_bwd: dtype must be f32 or bf16");
    const int vec = D % 4 == 0 && (reinterpret_cast<uintptr_t>(dW) & 15u) == 0;
    if (N == 0) {
        if (!accumulate) {  // every row absent
            hipLaunchKernelGGL(embed_zero_absent_k, dim3(static_cast<unsigned>((V + 3) / 4)), dim3(256), 0, s, nullptr,
                               0, V, dW, D, vec);
            AIC_LAUNCH_CHECK("embed_zero_absent");
        }
        return;
    }
    const size_t es = dtype_size(dt);
    // the run-list path: a chunk of 64 lanes x LB bytes divides the row, LB = 16, 8 or 4
    const int64_t row_bytes = D * static_cast<int64_t>(es);
    int lb = 0;
    for (int b : {16, 8, 4})
        if (!lb && row_bytes % (64 * b) == 0 && (reinterpret_cast<uintptr_t>(dout) % b) == 0) lb = b;
    const bool runs = lb > 0 && vec;
    auto* sk = static_cast<unsigned long long*>(stream_scratch(sizeof(unsigned long long) * N, s, 1));
    int* spos = static_cast<int*>(stream_scratch(sizeof(int) * (4 * N + 3), s));
    int* sid = spos + N;
    int* rstart = sid + N;      // N + 1 entries
    int* counts = rstart + N + 1;  // nruns, long runs
    int* lruns = counts + 2;
    const int n = static_cast<int>(N);
    hipLaunchKernelGGL(embed_chunk_sort_k, dim3(static_cast<unsigned>((N + kSortChunk - 1) / kSortChunk)), dim3(1024),
                       0, s, ids, n, V, sk);
    AIC_LAUNCH_CHECK("embed_chunk_sort");
    hipLaunchKernelGGL(embed_merge_rank_k, dim3(static_cast<unsigned>((N + 255) / 256)), dim3(256), 0, s, sk, n, spos,
                       sid);
    AIC_LAUNCH_CHECK("embed_merge_rank");
    if (!accumulate) {
        hipLaunchKernelGGL(embed_zero_absent_k, dim3(static_cast<unsigned>((V + 3) / 4)), dim3(256), 0, s, sid, n, V,
                           dW, D, vec);
        AIC_LAUNCH_CHECK("embed_zero_absent");
    }
    if (runs) {
        hipLaunchKernelGGL(embed_runs_k, dim3(1), dim3(1024), 0, s, sid, n, V, rstart, lruns, counts);
        AIC_LAUNCH_CHECK("embed_runs");
        // a wave per (run, chunk) (16 per block), at most 2048 blocks striding
        const int64_t items = N * (row_bytes / (64 * lb));
        AIC_CHECK(items < (1LL << 31), InvalidArgument, "embed_bwd: tokens x row chunks exceeds 2^31");
        const unsigned g = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(2048, (items + 15) / 16)));
        const int acc = accumulate ? 1 : 0;
        auto launch = [&](auto tag, auto lbc) {
            using T = decltype(tag);
            hipLaunchKernelGGL((embed_run_k<T, decltype(lbc)::value>), dim3(g), dim3(1024), 0, s, spos, sid, rstart,
                               lruns, counts, static_cast<const T*>(dout), D, dW, acc);
        };
        auto by_lb = [&](auto tag) {
            if (lb == 16) launch(tag, std::integral_constant<int, 16>{});
            else if (lb == 8) launch(tag, std::integral_constant<int, 8>{});
            else launch(tag, std::integral_constant<int, 4>{});
        };
        if (dt == DType::Float32) by_lb(float{});
        else by_lb(bf16{});
        AIC_LAUNCH_CHECK("embed_run");
        return;
    }
    const unsigned gy = static_cast<unsigned>(std::min<int64_t>((D + 63) / 64, 32));
    if (dt == DType::Float32)
        hipLaunchKernelGGL(embed_seg_k<float>, dim3(static_cast<unsigned>(N), gy), dim3(256), 0, s, spos, sid,
                           static_cast<int>(N), V, static_cast<const float*>(dout), D, dW, accumulate ? 1 : 0);
    else
        hipLaunchKernelGGL(embed_seg_k<bf16>, dim3(static_cast<unsigned>(N), gy), dim3(256), 0, s, spos, sid,
                           static_cast<int>(N), V, static_cast<const bf16*>(dout), D, dW, accumulate ? 1 : 0);
    AIC_LAUNCH_CHECK("embed_seg");
}

}  // namespace aic::hip
