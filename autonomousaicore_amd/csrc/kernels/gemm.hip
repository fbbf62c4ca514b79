// GEMM for the Linear layers: C = alpha * op(A) op(B) + beta * C + R.
//
// Replaces the reference's GEMM backend (src/cuda/cuda_gemm.cu:241-398, called from
// src/ops/matmul.cpp:25-52): one launch per product instead of one per batch slice, no
// weight transpose copy (op() reads either layout), fp32 accumulation, and the residual add
// of TransformerBlock (include/nn/transformer_block.hpp:26-36) fused into the epilogue.
//
// This file holds the dispatch (tile shape, split-K, grouped and expert-ragged launches), the
// split-K reduction and the SIMT kernel; the bf16 MFMA kernels are in gemm_kernels.inc,
// instantiated per operand layout and output type by gemm_{nt,nn,tn,tt}_{bf16,f32}.hip.
// fp32 path (the fp32 reference configuration) and odd shapes: a plain SIMT tiled kernel.
#include "gemm.hpp"

#include <algorithm>
#include <vector>
#include <type_traits>

#include "common.hpp"
#include "gemm_launch.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The 256-thread block's sum of every thread's (acc, nf) into *out / *out_nf: a fixed butterfly
// within each wave, then the four waves in order.  Every thread of the block must call it.
__device__ __forceinline__ void sq_block256(double acc, int nf, double* out, int* out_nf) {
    __shared__ double sd[4];
    __shared__ int sn[4];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        acc += __shfl_xor(acc, o);
        nf |= __shfl_xor(nf, o);
    }
    if ((threadIdx.x & 63) == 0) {
        sd[threadIdx.x >> 6] = acc;
        sn[threadIdx.x >> 6] = nf;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        *out = ((sd[0] + sd[1]) + sd[2]) + sd[3];
        *out_nf = sn[0] | sn[1] | sn[2] | sn[3];
    }
}

__device__ __forceinline__ void sq_add1(double& acc, int& nf, float v) {
    acc += static_cast<double>(v * v);
    nf |= (__float_as_uint(v) & 0x7f800000u) == 0x7f800000u;
}

// C = alpha * sum_z P[z] + beta * C + R over the split-K partials P [splits][M][N] (fp32,
// summed in z order: deterministic); with sq, each block also writes the sum of squares of
// the values it stored (one slot per block).
template <typename CT>
__global__ __launch_bounds__(256) void splitk_reduce_k(const float* __restrict__ P, int splits, int64_t pz, int M, int N,
                                                       float alpha, float beta, CT* C, int64_t ldc, const CT* R,
                                                       int64_t ldr, double* sq, int* sq_nf) {
    const int64_t total = static_cast<int64_t>(M) * N;
    double sqa = 0.0;
    int sqf = 0;
    for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int m = static_cast<int>(i / N), n = static_cast<int>(i % N);
        float acc = P[i];
        int z = 1;
        // eight loads in flight, added in z order
        for (; z + 8 <= splits; z += 8) {
            float p[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) p[u] = P[(z + u) * pz + i];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += p[u];
        }
        for (; z < splits; ++z) acc += P[z * pz + i];
        const int64_t ci = static_cast<int64_t>(m) * ldc + n;
        float v = alpha * acc;
        if (beta != 0.0f) v += beta * ld(C, ci);
        if (R) v += ld(R, static_cast<int64_t>(m) * ldr + n);
        st(C, ci, v);
        if (sq) sq_add1(sqa, sqf, v);  // fp32 C: the stored value
    }
    if (sq) sq_block256(sqa, sqf, sq + blockIdx.x, sq_nf + blockIdx.x);
}

// Sums of squares of the fp32 matrix C [M, N] (leading dimension ldc), one slot per block: the
// products whose path has no such epilogue.
__global__ __launch_bounds__(256) void sq_matrix_k(const float* __restrict__ C, int64_t ldc, int M, int N, double* sq,
                                                   int* sq_nf) {
    const int64_t total = static_cast<int64_t>(M) * N;
    double sqa = 0.0;
    int sqf = 0;
    for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256)
        sq_add1(sqa, sqf, C[(i / N) * ldc + i % N]);
    sq_block256(sqa, sqf, sq + blockIdx.x, sq_nf + blockIdx.x);
}

// ---------------------------------------------------------------------------------------
// SIMT tiled GEMM (fp32 configuration, odd shapes).  64x64 tile, 256 threads, 4x4 each.
// ---------------------------------------------------------------------------------------
template <typename T, typename CT>
__global__ __launch_bounds__(256) void gemm_simt(const T* __restrict__ A, const T* __restrict__ B, CT* C,
                                                  const CT* R, int64_t lda, int64_t ldb, int64_t ldc, int64_t ldr,
                                                  int M, int N, int K, int ta, int tb, float alpha, float beta) {
    constexpr int TS = 64, TK = 16;
    __shared__ float As[TK][TS + 4];
    __shared__ float Bs[TK][TS + 4];
    const int m0 = blockIdx.y * TS, n0 = blockIdx.x * TS;
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += TK) {
        for (int e = threadIdx.x; e < TS * TK; e += 256) {
            const int r = e / TK, kk = e % TK;
            const int m = m0 + r, k = k0 + kk;
            float a = 0.0f;
            if (m < M && k < K) a = ld(A, ta ? static_cast<int64_t>(k) * lda + m : static_cast<int64_t>(m) * lda + k);
            As[kk][r] = a;
            const int n = n0 + r;
            float b = 0.0f;
            if (n < N && k < K) b = ld(B, tb ? static_cast<int64_t>(n) * ldb + k : static_cast<int64_t>(k) * ldb + n);
            Bs[kk][r] = b;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < TK; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n >= N) continue;
            const int64_t ci = static_cast<int64_t>(m) * ldc + n;
            float v = alpha * acc[i][j];
            if (beta != 0.0f) v += beta * ld(C, ci);
            if (R) v += ld(R, static_cast<int64_t>(m) * ldr + n);
            st(C, ci, v);
        }
    }
}

template <int BM, int BN, int BK, int S, typename CT>
void dispatch_ragged(const RaggedArgs& r, hipStream_t s) {
    if (r.ragged_k) gemm_impl::launch_dma_ragged<BM, BN, BK, S, true, false, CT>(r, s);
    else if (r.g.transB) gemm_impl::launch_dma_ragged<BM, BN, BK, S, false, true, CT>(r, s);
    else gemm_impl::launch_dma_ragged<BM, BN, BK, S, false, false, CT>(r, s);
}

template <int BM, int BN, int BK, int S, typename CT>
void dispatch_grouped(const GemmArgs* a, int n, hipStream_t s) {
    if (!a[0].transA && a[0].transB) gemm_impl::launch_dma_grouped<BM, BN, BK, S, false, true, CT>(a, n, s);
    else if (!a[0].transA && !a[0].transB) gemm_impl::launch_dma_grouped<BM, BN, BK, S, false, false, CT>(a, n, s);
    else if (a[0].transA && !a[0].transB) gemm_impl::launch_dma_grouped<BM, BN, BK, S, true, false, CT>(a, n, s);
    else gemm_impl::launch_dma_grouped<BM, BN, BK, S, true, true, CT>(a, n, s);
}

template <int BM, int BN, int BK, int S, typename CT>
void dispatch_dma(const GemmArgs& a, hipStream_t s, int splits = 1, float* part = nullptr) {
    if (!a.transA && a.transB) gemm_impl::launch_dma<BM, BN, BK, S, false, true, CT>(a, s, splits, part);
    else if (!a.transA && !a.transB) gemm_impl::launch_dma<BM, BN, BK, S, false, false, CT>(a, s, splits, part);
    else if (a.transA && !a.transB) gemm_impl::launch_dma<BM, BN, BK, S, true, false, CT>(a, s, splits, part);
    else gemm_impl::launch_dma<BM, BN, BK, S, true, true, CT>(a, s, splits, part);
}

template <int BM, int BN, typename CT>
void dispatch_trans(const GemmArgs& a, hipStream_t s) {
    if (!a.transA && a.transB) gemm_impl::launch_mfma<BM, BN, false, true, CT>(a, s);
    else if (!a.transA && !a.transB) gemm_impl::launch_mfma<BM, BN, false, false, CT>(a, s);
    else if (a.transA && !a.transB) gemm_impl::launch_mfma<BM, BN, true, false, CT>(a, s);
    else gemm_impl::launch_mfma<BM, BN, true, true, CT>(a, s);
}

template <typename T, typename CT>
void launch_simt(const GemmArgs& a, hipStream_t s) {
    dim3 grid(static_cast<unsigned>((a.N + 63) / 64), static_cast<unsigned>((a.M + 63) / 64));
    hipLaunchKernelGGL((gemm_simt<T, CT>), grid, dim3(256), 0, s, static_cast<const T*>(a.A),
                       static_cast<const T*>(a.B), static_cast<CT*>(a.C), static_cast<const CT*>(a.R), a.lda, a.ldb,
                       a.ldc, a.ldr, static_cast<int>(a.M), static_cast<int>(a.N), static_cast<int>(a.K), a.transA,
                       a.transB, a.alpha, a.beta);
    AIC_LAUNCH_CHECK("gemm_simt");
}

}  // namespace

bool gemm_mfma_eligible(const GemmArgs& a) {
    if (a.ab != DType::BFloat16) return false;
    if (a.K % 8 || a.lda % 8 || a.ldb % 8 || !aligned16(a.A) || !aligned16(a.B)) return false;
    if (a.transA && a.M % 8) return false;
    if (!a.transB && a.N % 8) return false;
    return true;
}

bool gemm_q4_eligible(const GemmArgs& a) {
    if (!a.Bq || !a.Bscale || a.ab != DType::BFloat16 || a.transA) return false;
    if (a.K <= 0 || a.K % 64 || a.M < 8 || a.N < 8 || a.lda % 8 || !aligned16(a.A) || !aligned16(a.Bq)) return false;
    if (a.scale_t != DType::Float16 || reinterpret_cast<uintptr_t>(a.Bscale) % 4) return false;
    if (a.group <= 0 || a.group % 64 || a.group >= (int64_t{1} << 31) || a.ldb % 64) return false;
    if (!a.transB && (a.N % 64 || a.ldb < a.N)) return false;
    if (a.transB && a.ldb < a.K) return false;
    const int64_t rows = a.transB ? a.N : a.K;
    return rows * a.ldb / 64 < (int64_t{1} << 32);
}

bool gemm_dma_eligible(const GemmArgs& a) {
    if (!gemm_mfma_eligible(a)) return false;
    if (a.K % 64 || a.M < 8 || a.N < 8) return false;
    if (a.lda >= (int64_t{1} << 23) || a.ldb >= (int64_t{1} << 23)) return false;  // 32-bit copy offsets
    return true;
}

namespace {

// C = alpha * (sum of the split-K partials) + beta * C + R (and the sums of squares of C when
// a.sq_part is set: at most 1024 slots).
void splitk_reduce(const float* part, int splits, const GemmArgs& a, hipStream_t s) {
    const int64_t total = a.M * a.N;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, a.sq_part ? 1024 : 4096));
    if (a.c == DType::Float32) {
        AIC_CHECK(!a.sq_part || (a.sq_nf && grid <= a.sq_cap), InvalidArgument, "GEMM sums of squares: ", grid,
                  " slots needed, ", a.sq_cap, " given");
        hipLaunchKernelGGL(splitk_reduce_k<float>, dim3(grid), dim3(256), 0, s, part, splits, total,
                           static_cast<int>(a.M), static_cast<int>(a.N), a.alpha, a.beta, static_cast<float*>(a.C),
                           a.ldc, static_cast<const float*>(a.R), a.ldr, a.sq_part, a.sq_nf);
    } else {
        hipLaunchKernelGGL(splitk_reduce_k<bf16>, dim3(grid), dim3(256), 0, s, part, splits, total,
                           static_cast<int>(a.M), static_cast<int>(a.N), a.alpha, a.beta, static_cast<bf16*>(a.C),
                           a.ldc, static_cast<const bf16*>(a.R), a.ldr, nullptr, nullptr);
    }
    AIC_LAUNCH_CHECK("splitk_reduce_k");
}

// The sums of squares of the product already in C, for the paths without them in an epilogue.
void sq_matrix(const GemmArgs& a, hipStream_t s) {
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>({(a.M * a.N + 1023) / 1024, 256, a.sq_cap}));
    AIC_CHECK(a.sq_nf && grid >= 1, InvalidArgument, "GEMM sums of squares: no slots given");
    hipLaunchKernelGGL(sq_matrix_k, dim3(grid), dim3(256), 0, s, static_cast<const float*>(a.C), a.ldc,
                       static_cast<int>(a.M), static_cast<int>(a.N), a.sq_part, a.sq_nf);
    AIC_LAUNCH_CHECK("sq_matrix_k");
}

// Whether the rank term alpha X2 Y2^T fits the k-loop tail of the DMA kernels with BN-wide tiles.
bool rank_tail_ok(const GemmArgs& a, int64_t bn) {
    return a.r2 % 8 == 0 && a.ldx2 % 8 == 0 && aligned16(a.X2) && (a.y2_kmajor || (a.ldy2 % 8 == 0 && aligned16(a.Y2))) &&
           (a.seg_n == 0 || a.seg_n % bn == 0);
}

// C = alpha X2 Y2^T + C, per segment, as ordinary GEMMs (the shapes the kernel tail cannot take).
void rank_term_separately(const GemmArgs& a, hipStream_t s) {
    const size_t es = dtype_size(a.ab), ec = dtype_size(a.c);
    const int64_t nseg = a.seg_n > 0 ? a.N / a.seg_n : 1, nn = a.seg_n > 0 ? a.seg_n : a.N;
    for (int64_t g = 0; g < nseg; ++g) {
        GemmArgs t;
        t.transA = 0;
        t.transB = a.y2_kmajor ? 0 : 1;
        t.M = a.M;
        t.N = nn;
        t.K = a.r2;
        t.alpha = a.alpha;
        t.beta = 1.0f;
        t.A = static_cast<const char*>(a.X2) + es * g * a.r2;
        t.lda = a.ldx2;
        t.B = a.y2_kmajor ? static_cast<const char*>(a.Y2) + es * g * nn
                          : static_cast<const char*>(a.Y2) + es * g * nn * a.ldy2;
        t.ldb = a.ldy2;
        t.C = static_cast<char*>(a.C) + ec * g * nn;
        t.ldc = a.ldc;
        t.ab = a.ab;
        t.c = a.c;
        gemm(t, s);
    }
}

}  // namespace

namespace {
// The product with an INT4 B operand; tile size as for the bf16 operands (two stages on both),
// never split along K.
void gemm_q4(const GemmArgs& a, hipStream_t s) {
    AIC_CHECK(gemm_q4_eligible(a), InvalidArgument,
              "INT4 GEMM: unsupported shape or layout (bf16 A, K % 64, group % 64, ldb % 64, N % 64 for dy W)");
    const int64_t t256 = ((a.M + 255) / 256) * ((a.N + 255) / 256);
    const bool big = t256 >= 128;
    if (a.r2 > 0) {
        const int64_t bn = big ? 256 : 128;
        if (!rank_tail_ok(a, bn)) {
            GemmArgs b = a;
            b.r2 = 0;
            gemm_q4(b, s);
            rank_term_separately(a, s);
            return;
        }
    }
    if (a.c == DType::Float32) {
        if (big) a.transB ? gemm_impl::launch_dma_q4<256, 256, 64, 2, true, float>(a, s)
                          : gemm_impl::launch_dma_q4<256, 256, 64, 2, false, float>(a, s);
        else a.transB ? gemm_impl::launch_dma_q4<128, 128, 64, 2, true, float>(a, s)
                      : gemm_impl::launch_dma_q4<128, 128, 64, 2, false, float>(a, s);
    } else {
        if (big) a.transB ? gemm_impl::launch_dma_q4<256, 256, 64, 2, true, bf16>(a, s)
                          : gemm_impl::launch_dma_q4<256, 256, 64, 2, false, bf16>(a, s);
        else a.transB ? gemm_impl::launch_dma_q4<128, 128, 64, 2, true, bf16>(a, s)
                      : gemm_impl::launch_dma_q4<128, 128, 64, 2, false, bf16>(a, s);
    }
}
}  // namespace

void gemm(const GemmArgs& a, hipStream_t s) {
    AIC_CHECK(a.M >= 0 && a.N >= 0 && a.K >= 0, InvalidArgument, "negative GEMM size");
    AIC_CHECK(a.M < (1LL << 31) && a.N < (1LL << 31) && a.K < (1LL << 31), InvalidArgument, "GEMM size too large");
    AIC_CHECK(a.A && (a.B || a.Bq) && a.C, InvalidArgument, "null GEMM operand");
    AIC_CHECK(a.ab == DType::Float32 || a.ab == DType::BFloat16, DTypeMismatch, "GEMM inputs must be f32 or bf16");
    AIC_CHECK(a.c == DType::Float32 || a.c == DType::BFloat16, DTypeMismatch, "GEMM output must be f32 or bf16");
    const int64_t amin = a.transA ? a.M : a.K, bmin = a.transB ? a.K : a.N;
    AIC_CHECK(a.lda >= (amin > 0 ? amin : 1) && a.ldb >= (bmin > 0 ? bmin : 1) && a.ldc >= (a.N > 0 ? a.N : 1),
              InvalidArgument, "leading dimension smaller than the row length");
    if (a.r2 > 0) {
        AIC_CHECK(a.X2 && a.Y2, InvalidArgument, "low-rank GEMM term without X2 / Y2");
        AIC_CHECK(a.seg_n >= 0 && (a.seg_n == 0 || a.N % a.seg_n == 0), InvalidArgument,
                  "low-rank segments must tile N");
        const int64_t segs = a.seg_n > 0 ? a.N / a.seg_n : 1;
        AIC_CHECK(a.ldx2 >= segs * a.r2 && a.ldy2 >= (a.y2_kmajor ? a.N : a.r2), InvalidArgument,
                  "low-rank term: leading dimension smaller than the row length");
    }
    if (a.M == 0 || a.N == 0) return;
    if (a.sq_part) {
        AIC_CHECK(a.c == DType::Float32 && a.sq_nf && a.sq_cap > 0 && !a.rope_cos && a.glu_f == 0 && !a.dglu_gu,
                  InvalidArgument, "GEMM sums of squares: fp32 output only, without the RoPE / SwiGLU epilogues");
        // in the DMA tile kernels' epilogue or split-K reduction; the other paths (INT4 B, a
        // low-rank term, the non-DMA kernels) read the product back
        if (a.Bq || a.r2 > 0 || !gemm_dma_eligible(a)) {
            GemmArgs b = a;
            b.sq_part = nullptr;
            b.sq_nf = nullptr;
            b.sq_cap = 0;
            gemm(b, s);
            sq_matrix(a, s);
            return;
        }
    }
    if (a.rope_cos) {
        AIC_CHECK(a.rope_sin && a.rope_hd > 0 && a.rope_hd % 2 == 0 && a.rope_cols % a.rope_hd == 0 &&
                      a.rope_cols <= a.N && a.rope_seq > 0 && a.M % a.rope_seq == 0 && a.beta == 0.0f && !a.R,
                  InvalidArgument, "GEMM rotary epilogue: bad rope arguments");
        // in the epilogue: bf16 output on full 256x256 tiles, for the eight-wave plain path heads of
        // 128 (split in halves by the 64-column wave sub-tiles, exchanged through LDS) or 64 (one
        // per wave sub-tile), for the four-wave INT4 path heads of 128 (one per wave sub-tile,
        // after the kernel's low-rank term)
        const bool tiles = a.c == DType::BFloat16 && a.M % 256 == 0 && a.N % 256 == 0 && a.rope_cols % 256 == 0 &&
                           a.ldc % 8 == 0 && aligned16(a.C) && ((a.M / 256) * (a.N / 256) >= 128);
        const bool fused = tiles && (a.Bq ? a.rope_hd == 128 && a.transB && gemm_q4_eligible(a) &&
                                                (a.r2 == 0 || rank_tail_ok(a, 256))
                                          : (a.rope_hd == 128 || a.rope_hd == 64) && gemm_impl::kDmaWaves256 == 8 &&
                                                gemm_dma_eligible(a) && a.r2 == 0);
        if (!fused) {
            GemmArgs b = a;
            b.rope_cos = b.rope_sin = nullptr;
            if (a.Bq && !gemm_q4_eligible(a)) {
                // an INT4 weight the operand-load dequantization cannot take (group or row length
                // not a multiple of 64, misaligned scales): dequantized into a scratch copy first
                const int64_t nw = a.N * a.K;
                AIC_CHECK(a.transB && a.ldb == a.K && a.Bscale, InvalidArgument,
                          "INT4 GEMM: the weight must be [N][K] with ld K");
                void* w = stream_scratch(dtype_size(a.ab) * static_cast<size_t>(nw), s, 5);
                int4_dequant(a.Bq, a.Bscale, a.scale_t, nw, a.group, w, a.ab, s);
                b.B = w;
                b.Bq = nullptr;
                b.Bscale = nullptr;
            }
            gemm(b, s);
            rope(a.C, a.ldc, a.M / a.rope_seq, a.rope_seq, a.rope_cols / a.rope_hd, a.rope_hd, a.rope_start,
                 a.rope_cos, a.rope_sin, false, a.c, s);
            return;
        }
    }
    if (a.glu_f > 0) {
        AIC_CHECK(a.N == 2 * a.glu_f && a.glu_out && a.ld_glu >= a.glu_f && a.beta == 0.0f && !a.R && !a.rope_cos,
                  InvalidArgument, "GEMM SwiGLU epilogue: bad arguments");
        // in the epilogue: bf16 x W^T on full 256x256 tiles of the eight-wave plain path, or of the
        // four-wave INT4 path (also after its low-rank term, whose segments follow the pairing)
        const bool tiles = a.transB && !a.transA && a.c == DType::BFloat16 && a.M % 256 == 0 && a.glu_f % 128 == 0 &&
                           a.ldc % 8 == 0 && aligned16(a.C) && a.ld_glu % 8 == 0 && aligned16(a.glu_out) &&
                           ((a.M / 256) * (a.N / 256) >= 128);
        const bool fused = tiles && (a.Bq ? gemm_q4_eligible(a) && (a.r2 == 0 || rank_tail_ok(a, 256))
                                          : gemm_impl::kDmaWaves256 == 8 && gemm_dma_eligible(a) && a.r2 == 0);
        if (!fused) {
            GemmArgs b = a;
            b.glu_f = 0;
            b.glu_out = nullptr;
            gemm(b, s);
            swiglu_fwd(a.C, static_cast<const char*>(a.C) + dtype_size(a.c) * a.glu_f, a.ldc, a.glu_out, a.ld_glu,
                       a.M, a.glu_f, a.c, s);
            return;
        }
        if (a.Bq) gemm_q4(a, s);
        else dispatch_dma<256, 256, 64, 2, bf16>(a, s);
        return;
    }
    if (a.dglu_gu) {
        AIC_CHECK(a.dglu_out && a.dglu_ld >= 2 * a.N && a.beta == 0.0f && !a.R && !a.rope_cos && a.glu_f == 0,
                  InvalidArgument, "GEMM SwiGLU-backward epilogue: bad arguments");
        // in the epilogue of the full-tile paths without K split (at least 128 tiles of 256x256)
        const int64_t es = static_cast<int64_t>(dtype_size(a.c));
        const bool fused = a.c == DType::BFloat16 && (a.Bq ? gemm_q4_eligible(a) : gemm_dma_eligible(a)) &&
                           a.M % 256 == 0 && a.N % 256 == 0 &&
                           (a.M / 256) * (a.N / 256) >= 128 && a.ldc % 8 == 0 && aligned16(a.C) &&
                           a.dglu_ld % 8 == 0 && aligned16(a.dglu_gu) && aligned16(a.dglu_out) &&
                           (a.r2 == 0 || rank_tail_ok(a, 256));  // C is not written: no rank term added later
        if (!fused) {
            GemmArgs b = a;
            b.dglu_gu = nullptr;
            b.dglu_out = nullptr;
            gemm(b, s);
            swiglu_bwd(a.dglu_gu, static_cast<const char*>(a.dglu_gu) + es * a.N, a.dglu_ld, a.C, a.ldc, a.dglu_out,
                       static_cast<char*>(a.dglu_out) + es * a.N, a.dglu_ld, a.M, a.N, a.c, s);
            return;
        }
    }
    if (a.Bq) {
        gemm_q4(a, s);
        return;
    }
    if (gemm_dma_eligible(a)) {
        // 256x256 tiles from half a round of tiles up (measured on the 1B shapes: 176 tiles of
        // 256x256 beat 704 of 128x128 by 24%); between 32 and 128 of them over a long K, 256x256
        // tiles with K split so that about one full round runs (the 2048x2048x8192 weight
        // gradient: 80 us against 93 us on 128x128 tiles)
        const int64_t t256 = ((a.M + 255) / 256) * ((a.N + 255) / 256);
        const int64_t t128 = ((a.M + 127) / 128) * ((a.N + 127) / 128);
        const int64_t tw = ((a.M + 127) / 128) * ((a.N + 255) / 256);  // 128x256 tiles
        const bool big = t256 >= 128;
        // under a round of 256x256 tiles over a long K (a 1024-wide head's input gradient: 128
        // tiles, K 32000): split K until about one round runs (682 -> 444 us there)
        int splits256 = 1;
        if (a.r2 == 0 && t256 < 256 && t256 >= 32 && a.K >= 4096) {
            splits256 = static_cast<int>(std::min<int64_t>(4, 256 / t256));
            while (splits256 > 1 && a.K % (64LL * splits256)) --splits256;
        }
        if (a.r2 > 0) {
            const int64_t bn = big ? 256 : 128;
            if (!rank_tail_ok(a, bn)) {
                GemmArgs b = a;
                b.r2 = 0;
                gemm(b, s);
                rank_term_separately(a, s);
                return;
            }
        }
        // few output tiles over a long K: split K so that the launch fills the chip (partials
        // summed in a fixed order afterwards)
        if (splits256 > 1) {
            float* part = static_cast<float*>(stream_scratch(sizeof(float) * splits256 * a.M * a.N, s, 7));
            dispatch_dma<256, 256, 64, 2, float>(a, s, splits256, part);
            splitk_reduce(part, splits256, a, s);
            return;
        }
        int splits = 1;
        if (a.r2 == 0 && !big && t128 < 128 && a.K >= 1024) {
            splits = static_cast<int>(std::min<int64_t>({a.K / 512, (256 + t128 - 1) / t128, 16}));
            while (splits > 1 && a.K % (64LL * splits)) --splits;
        }
        if (splits > 1) {
            float* part = static_cast<float*>(stream_scratch(sizeof(float) * splits * a.M * a.N, s, 7));
            dispatch_dma<128, 128, 64, 4, float>(a, s, splits, part);
            splitk_reduce(part, splits, a, s);
            return;
        }
        // under a round of 256x256 tiles where 128x256 tiles fill between half the chip and one
        // round (768- and 1024-wide products over 8192 rows): one round of the four-wave 128x256
        // kernel beats a partial round of 256x256 tiles and two rounds of 128x128 ones (measured
        // 3-9% on those shapes); with a residual and at least half a round of 256x256 tiles the
        // persistent kernel stays ahead (its epilogue overlaps the next tile's copies)
        if (a.r2 == 0 && !a.rope_cos && !a.dglu_gu && t256 < 256 && tw >= 128 && tw <= 256 && !(a.R && big)) {
            if (a.c == DType::Float32) dispatch_dma<128, 256, 64, 3, float>(a, s);
            else dispatch_dma<128, 256, 64, 3, bf16>(a, s);
            return;
        }
        if (a.c == DType::Float32) {
            if (big) dispatch_dma<256, 256, 64, 2, float>(a, s);
            else dispatch_dma<128, 128, 64, 4, float>(a, s);
        } else {
            if (big) dispatch_dma<256, 256, 64, 2, bf16>(a, s);
            else dispatch_dma<128, 128, 64, 4, bf16>(a, s);
        }
        return;
    }
    if (a.r2 > 0) {
        GemmArgs b = a;
        b.r2 = 0;
        gemm(b, s);
        rank_term_separately(a, s);
        return;
    }
    if (gemm_mfma_eligible(a)) {
        const bool big = a.M >= 2048 && a.N >= 2048 && ((a.M / 256) * (a.N / 256) >= 256);
        if (a.c == DType::Float32) {
            if (big) dispatch_trans<256, 256, float>(a, s);
            else dispatch_trans<128, 128, float>(a, s);
        } else {
            if (big) dispatch_trans<256, 256, bf16>(a, s);
            else dispatch_trans<128, 128, bf16>(a, s);
        }
        return;
    }
    if (a.ab == DType::Float32) {
        if (a.c == DType::Float32) launch_simt<float, float>(a, s);
        else launch_simt<float, bf16>(a, s);
    } else {
        if (a.c == DType::Float32) launch_simt<bf16, float>(a, s);
        else launch_simt<bf16, bf16>(a, s);
    }
}

void gemm_grouped(const GemmArgs* a, int n, hipStream_t s) {
    AIC_CHECK(a && n >= 0, InvalidArgument, "gemm_grouped: bad arguments");
    bool one_launch = n >= 2 && n <= gemm_impl::kMaxGroups;
    int64_t t256 = 0;
    for (int i = 0; i < n && one_launch; ++i) {
        const GemmArgs& x = a[i];
        one_launch = gemm_dma_eligible(x) && x.transA == a[0].transA && x.transB == a[0].transB &&
                     x.ab == a[0].ab && x.c == a[0].c && !x.R && x.r2 == 0 && x.alpha == a[0].alpha &&
                     x.beta == a[0].beta && x.M > 0 && x.N > 0 && x.ldc >= x.N &&
                     x.lda >= (x.transA ? x.M : x.K) && x.ldb >= (x.transB ? x.K : x.N);
        t256 += ((x.M + 255) / 256) * ((x.N + 255) / 256);
    }
    if (!one_launch) {
        for (int i = 0; i < n; ++i) {
            GemmArgs b = a[i];
            if (a[0].sq_part) {  // the launch's slot region in equal shares
                const int64_t share = a[0].sq_cap / n;
                b.sq_part = a[0].sq_part + i * share;
                b.sq_nf = a[0].sq_nf + i * share;
                b.sq_cap = share;
            } else {
                b.sq_part = nullptr;
            }
            gemm(b, s);
        }
        return;
    }
    if (t256 > 256 && t256 % 256 != 0 && t256 % 256 <= 64) {
        // A few tiles past whole rounds of the chip (the 1B layer's four weight gradients: 784
        // tiles of 256x256, 3 rounds + 16) would cost most of a fourth round.  One product gives
        // up whole tile-columns (or tile-rows) making up the excess; they run after the launch
        // as their own GEMM, which splits them along K over the chip (834 -> 745 us at that
        // shape).  Taken only when the remaining tiles fall evenly on the 8 XCDs (block b runs
        // on XCD b % 8; each product's blocks start at a multiple of 8).
        const int64_t excess = t256 % 256, rounds = t256 / 256;
        for (int i = n - 1; i >= 0; --i) {
            const GemmArgs& x = a[i];
            const int64_t tm = (x.M + 255) / 256, tn = (x.N + 255) / 256;
            GemmArgs keep = x, cut = x;
            const size_t es = dtype_size(x.ab), ec = dtype_size(x.c);
            if (excess % tm == 0 && excess / tm < tn) {  // the rightmost tile-columns
                const int64_t n0 = 256 * (tn - excess / tm);
                keep.N = n0;
                cut.N = x.N - n0;
                cut.B = static_cast<const char*>(x.B) + es * (x.transB ? n0 * x.ldb : n0);
                cut.C = static_cast<char*>(x.C) + ec * n0;
            } else if (excess % tn == 0 && excess / tn < tm) {  // the bottom tile-rows
                const int64_t m0 = 256 * (tm - excess / tn);
                keep.M = m0;
                cut.M = x.M - m0;
                cut.A = static_cast<const char*>(x.A) + es * (x.transA ? m0 : m0 * x.lda);
                cut.C = static_cast<char*>(x.C) + ec * m0 * x.ldc;
            } else {
                continue;
            }
            std::vector<GemmArgs> g(a, a + n);
            g[i] = keep;
            int64_t per_xcd[8] = {};
            for (const GemmArgs& y : g) {
                const int64_t t = ((y.M + 255) / 256) * ((y.N + 255) / 256);
                for (int xcd = 0; xcd < 8; ++xcd) per_xcd[xcd] += t / 8 + (xcd < t % 8 ? 1 : 0);
            }
            if (*std::max_element(per_xcd, per_xcd + 8) > 32 * rounds) continue;
            if (g[0].c == DType::Float32) dispatch_grouped<256, 256, 64, 2, float>(g.data(), n, s);
            else dispatch_grouped<256, 256, 64, 2, bf16>(g.data(), n, s);
            cut.sq_part = nullptr;
            if (a[0].sq_part) {  // the launch's blocks (8-aligned per product), then the cut's slots
                int64_t blocks = 0;
                for (const GemmArgs& y : g) blocks += (((y.M + 255) / 256) * ((y.N + 255) / 256) + 7) / 8 * 8;
                AIC_CHECK(blocks < a[0].sq_cap, InvalidArgument, "grouped GEMM sums of squares: region too small");
                cut.sq_part = a[0].sq_part + blocks;
                cut.sq_nf = a[0].sq_nf + blocks;
                cut.sq_cap = a[0].sq_cap - blocks;
            }
            gemm(cut, s);
            return;
        }
    }
    // under half a round of 256x256 tiles: 128x128 tiles, or 128x256 ones where those fill one
    // round and 128x128 tiles would need more (the 125M layer's four weight gradients: 216 tiles
    // of 128x256 against 432 of 128x128)
    int64_t t128 = 0, tw = 0;
    for (int i = 0; i < n; ++i) {
        t128 += ((a[i].M + 127) / 128) * ((a[i].N + 127) / 128);
        tw += ((a[i].M + 127) / 128) * ((a[i].N + 255) / 256);
    }
    const bool wide = t256 < 128 && t128 > 256 && tw <= 256;
    if (a[0].c == DType::Float32) {
        if (t256 >= 128) dispatch_grouped<256, 256, 64, 2, float>(a, n, s);
        else if (wide) dispatch_grouped<128, 256, 64, 3, float>(a, n, s);
        else dispatch_grouped<128, 128, 64, 4, float>(a, n, s);
    } else {
        if (t256 >= 128) dispatch_grouped<256, 256, 64, 2, bf16>(a, n, s);
        else if (wide) dispatch_grouped<128, 256, 64, 3, bf16>(a, n, s);
        else dispatch_grouped<128, 128, 64, 4, bf16>(a, n, s);
    }
}

// One product: the tile kernels write one slot per block (at most its 128x128 tile count,
// rounded up to a multiple of 8 for the grouped launch's per-product padding), the split-K
// reduction at most 1024 and the read-back pass at most 256.  Several products: the grouped
// launch's blocks, or the blocks of all but a cut product plus the cut's own launch, or equal
// shares of the region per product (one gemm() each) -- all within n + 1 times the largest
// single bound.
int64_t gemm_sq_slots(const GemmArgs* a, int n) {
    AIC_CHECK(a && n >= 1, InvalidArgument, "gemm_sq_slots: no products");
    int64_t most = 0;
    for (int i = 0; i < n; ++i) {
        const int64_t t128 = ((a[i].M + 127) / 128) * ((a[i].N + 127) / 128);
        most = std::max(most, (std::max<int64_t>(t128, 1024) + 7) / 8 * 8);
    }
    return n == 1 ? most : (n + 1) * most;
}

// The ragged-K launch writes one slot per block: E experts of its tile count rounded up to a
// multiple of 8 (256x256 or 128x128 tiles); the fallback (one product per expert, in grouped
// launches of up to 8 sharing the region equally) needs its launches' bounds.
int64_t gemm_ragged_sq_slots(int64_t M, int64_t N, int E) {
    AIC_CHECK(M > 0 && N > 0 && E >= 1, InvalidArgument, "gemm_ragged_sq_slots: bad shape");
    const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
    GemmArgs g;
    g.M = M;
    g.N = N;
    std::vector<GemmArgs> eight(8, g);
    const int64_t launches = (E + 7) / 8;
    return std::max(E * ((t128 + 7) / 8 * 8), launches * gemm_sq_slots(eight.data(), std::min(E, 8)));
}

bool gemm_ragged_eligible(const RaggedArgs& r) {
    const GemmArgs& a = r.g;
    if (!r.offsets || r.E < 1 || r.E > 64 || a.R || a.r2 || a.ab != DType::BFloat16) return false;
    if (a.M < 8 || a.N < 8 || a.lda % 8 || a.ldb % 8 || !aligned16(a.A) || !aligned16(a.B)) return false;
    if (a.M > (int64_t{1} << 30) || a.N > (int64_t{1} << 30)) return false;
    if (r.ragged_k) {
        // A [rows][M], B [rows][N]: row offsets move both by whole rows
        return a.transA && !a.transB && a.M % 8 == 0 && a.N % 8 == 0 && a.lda >= a.M && a.ldb >= a.N &&
               a.ldc >= a.N && r.b_stride == 0 && r.c_stride >= a.M * a.ldc;
    }
    return !a.transA && a.K > 0 && a.K % 64 == 0 && a.lda >= a.K && a.ldc >= a.N && (a.transB || a.N % 8 == 0) &&
           a.ldb >= (a.transB ? a.K : a.N) && r.b_stride % 8 == 0;
}

void gemm_ragged(const RaggedArgs& r, hipStream_t s) {
    AIC_CHECK(gemm_ragged_eligible(r), InvalidArgument, "gemm_ragged: unsupported shape, layout or dtype");
    const GemmArgs& a = r.g;
    bool force256 = false;
    if (a.glu_f > 0 || a.dglu_gu) {
        // SwiGLU (forward or backward) of an expert-ragged product: in the epilogue on bf16 outputs
        // whose columns are whole 256-wide tiles (the forward on 256x256 tiles, whose columns pair
        // 128 gate with 128 up columns); otherwise the product, then the pass over all rows
        AIC_CHECK(!r.ragged_k && a.beta == 0.0f && !a.R && !(a.glu_f > 0 && a.dglu_gu), InvalidArgument,
                  "gemm_ragged: SwiGLU epilogue arguments");
        const bool cols = a.c == DType::BFloat16 && a.N % 256 == 0 && a.ldc % 8 == 0 && aligned16(a.C);
        const bool glu = a.glu_f > 0 && cols && a.transB && !a.transA && gemm_impl::kDmaWaves256 == 8 &&
                         a.N == 2 * a.glu_f && a.glu_f % 128 == 0 && a.ld_glu >= a.glu_f && a.ld_glu % 8 == 0 &&
                         aligned16(a.glu_out);
        const bool dglu = a.dglu_gu && cols && a.dglu_ld >= 2 * a.N && a.dglu_ld % 8 == 0 && aligned16(a.dglu_gu) &&
                          aligned16(a.dglu_out);
        if (!glu && !dglu) {
            RaggedArgs b = r;
            b.g.glu_f = 0;
            b.g.glu_out = nullptr;
            b.g.dglu_gu = nullptr;
            b.g.dglu_out = nullptr;
            gemm_ragged(b, s);
            const int64_t es = static_cast<int64_t>(dtype_size(a.c));
            if (a.glu_f > 0)
                swiglu_fwd(a.C, static_cast<const char*>(a.C) + es * a.glu_f, a.ldc, a.glu_out, a.ld_glu, a.M, a.glu_f,
                           a.c, s);
            else
                swiglu_bwd(a.dglu_gu, static_cast<const char*>(a.dglu_gu) + es * a.N, a.dglu_ld, a.C, a.ldc,
                           a.dglu_out, static_cast<char*>(a.dglu_out) + es * a.N, a.dglu_ld, a.M, a.N, a.c, s);
            return;
        }
        force256 = glu;
    }
    // Tile shape: the grid's tiles (a bound for ragged M) in rounds of 256 CUs; the 256x256
    // tile unless its last round leaves so many CUs idle that 128x128 tiles (taken as 0.8 of
    // its rate) fill the rounds better.
    auto tiles = [&](int64_t t) {
        const int64_t tn = (a.N + t - 1) / t;
        return r.ragged_k ? r.E * ((a.M + t - 1) / t) * tn : ((a.M + t - 1) / t + r.E) * tn;
    };
    auto fill = [](int64_t n) { return static_cast<double>(n) / (256.0 * static_cast<double>((n + 255) / 256)); };
    // bf16 rows on whole 256-column tiles run the persistent kernel (gemm_kernels.inc,
    // launch_dma_ragged), whose blocks take tile after tile: a round of 256 tiles is enough
    const bool pers = a.c == DType::BFloat16 && !r.ragged_k && r.E <= 63 && a.N % 256 == 0 && a.K % 128 == 0 &&
                      a.K >= 256 && a.beta == 0.0f;
    const bool big = force256 || (pers && tiles(256) >= 256) ||
                     (tiles(256) >= 128 && fill(tiles(256)) >= 0.8 * fill(tiles(128)));
    if (a.c == DType::Float32) {
        if (big) dispatch_ragged<256, 256, 64, 2, float>(r, s);
        else dispatch_ragged<128, 128, 64, 4, float>(r, s);
    } else {
        if (big) dispatch_ragged<256, 256, 64, 2, bf16>(r, s);
        else dispatch_ragged<128, 128, 64, 4, bf16>(r, s);
    }
}

}  // namespace aic::hip
