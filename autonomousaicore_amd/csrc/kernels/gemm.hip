// GEMM for the Linear layers: C = alpha * op(A) op(B) + beta * C + R.
//
// Replaces the reference's GEMM backend (src/cuda/cuda_gemm.cu:241-398, called from
// src/ops/matmul.cpp:25-52): one launch per product instead of one per batch slice, no
// weight transpose copy (op() reads either layout), fp32 accumulation, and the residual add
// of TransformerBlock (include/nn/transformer_block.hpp:26-36) fused into the epilogue.
//
// bf16 path: hand-written CDNA4 kernel on v_mfma_f32_32x32x16_bf16 (gemm_bf16_dma).
//   * 256 threads = 4 waves arranged 2x2; macro tile BM x BN x 64, each wave BM/2 x BN/2
//     built from 32x32 MFMA blocks; fp32 accumulators live in AGPRs.
//   * Operand tiles go from HBM straight into LDS with global_load_lds_dwordx4 (no VGPR
//     staging), S stages deep; a wave waits only for its own copies of the tile it is about
//     to read (s_waitcnt vmcnt(N)) and one s_barrier per K step publishes all waves' copies.
//   * An operand whose K dimension is contiguous in HBM is kept as [rows][64] in LDS with
//     16-byte chunks XOR-swizzled per row and read with ds_read_b128.  An operand whose
//     rows are contiguous (dgrad's weight, both wgrad operands) is kept untransposed as
//     [64][rows] and read with ds_read_b64_tr_b16, which transposes 4x4 blocks of 16-bit
//     values across each group of 16 lanes; its chunks are XOR-swizzled by 4*(k & 3).
//   * Blocks are remapped so that each XCD (hardware dispatches block b to XCD b % 8)
//     works on a contiguous, M-grouped range of tiles and shares A/B panels in its L2.
// Shapes the DMA kernel cannot take (K % 64 != 0) use gemm_bf16_mfma, which stages tiles
// through registers (and transposes row-contiguous operands there).
// fp32 path (the fp32 reference configuration) and odd shapes: a plain SIMT tiled kernel.
#include "gemm.hpp"

#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

constexpr int kBK = 64;

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

struct MfmaParams {
    const bf16* A;
    const bf16* B;
    void* C;
    const void* R;
    int64_t lda, ldb, ldc, ldr;
    int M, N, K;
    float alpha, beta;
    int vec;  // C (and R) rows allow 4-element vector access: ld % 4 == 0, 16-byte aligned base
    // low-rank term acc += X2 Y2^T (r2 % 8 == 0; 0: none); split-K: block z covers K rows
    // [z K, (z+1) K) of the operands and writes the fp32 partial C + z * cz
    const bf16* X2;
    const bf16* Y2;
    int64_t ldx2, ldy2, cz;
    int r2, seg_n, y2k;
};

// A grouped launch: up to kMaxGroups independent products of one kernel configuration, each
// with its own operands and sizes, in one grid.  Group g owns the blocks [tile0, tile0 +
// nblocks), nblocks its tile count rounded up to a multiple of 8 so that every group's block ids
// keep the XCD mapping (block b runs on XCD b % 8).
constexpr int kMaxGroups = 8;
struct GroupDesc {
    const bf16* A;
    const bf16* B;
    void* C;
    int64_t lda, ldb, ldc;
    int M, N, K;
    int tile0, nblocks;
};
struct DmaParams {
    MfmaParams p;
    int ngroups;  // 0: the single product of p
    GroupDesc g[kMaxGroups];
};

// Four consecutive elements of a C / R row, as floats.
__device__ __forceinline__ void ld4(const float* p, float v[4]) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}
__device__ __forceinline__ void ld4(const bf16* p, float v[4]) {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = __uint_as_float(t.x << 16); v[1] = __uint_as_float(t.x & 0xffff0000u);
    v[2] = __uint_as_float(t.y << 16); v[3] = __uint_as_float(t.y & 0xffff0000u);
}
__device__ __forceinline__ void st4(float* p, const float v[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st4(bf16* p, const float v[4]) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}

// Map the hardware block id to a tile so that consecutive tiles (same A row panel,
// neighbouring B panels) land on the same XCD.
__device__ __forceinline__ int xcd_id(int bid, int nb) {
    const int q = nb / 8, r = nb % 8;
    const int xcd = bid % 8, local = bid / 8;
    return (xcd < r) ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// Tile (tm, tn) of linear id (id < tiles_m * tiles_n): groups of 8 consecutive row tiles.
__device__ __forceinline__ void id_to_tile(int id, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int G = 8;
    const int per_group = G * tiles_n;
    const int group = id / per_group;
    const int first_m = group * G;
    const int gsize = min(tiles_m - first_m, G);
    const int inner = id % per_group;
    tm = first_m + inner % gsize;
    tn = inner / gsize;
}

__device__ __forceinline__ void tile_of(int bid, int nb, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int id = xcd_id(bid, nb);
    constexpr int G = 8;
    const int per_group = G * tiles_n;
    const int group = id / per_group;
    const int first_m = group * G;
    const int gsize = min(tiles_m - first_m, G);
    const int inner = id % per_group;
    tm = first_m + inner % gsize;
    tn = inner / gsize;
}

// Loads one ROWS x 64 operand tile whose K dimension is contiguous in HBM.
template <int ROWS>
struct KContigLoader {
    static constexpr int CH = ROWS * kBK / 8 / 256;  // 16-byte chunks per thread
    uint4 r[CH];
    __device__ __forceinline__ void load(const bf16* __restrict__ g, int64_t ld, int row0, int nrows, int k0, int K) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = threadIdx.x + 256 * i;
            const int row = c >> 3, kc = c & 7;
            const int gr = row0 + row, gk = k0 + kc * 8;
            if (gr < nrows && gk < K)
                r[i] = *reinterpret_cast<const uint4*>(g + static_cast<int64_t>(gr) * ld + gk);
            else
                r[i] = make_uint4(0, 0, 0, 0);
        }
    }
    __device__ __forceinline__ void store(bf16* s) const {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = threadIdx.x + 256 * i;
            const int row = c >> 3, kc = c & 7;
            *reinterpret_cast<uint4*>(s + row * kBK + ((kc ^ swz(row)) << 3)) = r[i];
        }
    }
};

// Loads one ROWS x 64 operand tile stored [K][ld] (rows contiguous in HBM) and transposes
// it in registers: thread t < ROWS owns the 8(k) x 8(row) block (kg = t % 8, rc = t / 8).
template <int ROWS>
struct RowContigLoader {
    uint4 r[8];
    __device__ __forceinline__ void load(const bf16* __restrict__ g, int64_t ld, int row0, int nrows, int k0, int K) {
        const int t = threadIdx.x;
        if (t >= ROWS) return;
        const int kg = t & 7, rc = t >> 3;
        const int gr = row0 + rc * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int gk = k0 + kg * 8 + i;
            if (gk < K && gr < nrows)
                r[i] = *reinterpret_cast<const uint4*>(g + static_cast<int64_t>(gk) * ld + gr);
            else
                r[i] = make_uint4(0, 0, 0, 0);
        }
    }
    __device__ __forceinline__ static uint32_t w(const uint4& v, int i) {
        return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
    }
    __device__ __forceinline__ void store(bf16* s) const {
        const int t = threadIdx.x;
        if (t >= ROWS) return;
        const int kg = t & 7, rc = t >> 3;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
            uint4 o;
            o.x = __builtin_amdgcn_perm(w(r[1], j >> 1), w(r[0], j >> 1), sel);
            o.y = __builtin_amdgcn_perm(w(r[3], j >> 1), w(r[2], j >> 1), sel);
            o.z = __builtin_amdgcn_perm(w(r[5], j >> 1), w(r[4], j >> 1), sel);
            o.w = __builtin_amdgcn_perm(w(r[7], j >> 1), w(r[6], j >> 1), sel);
            const int row = rc * 8 + j;
            *reinterpret_cast<uint4*>(s + row * kBK + ((kg ^ swz(row)) << 3)) = o;
        }
    }
};

template <int BM, int BN, bool TA, bool TB, typename CT>
__global__ __launch_bounds__(256, 1) void gemm_bf16_mfma(const MfmaParams p) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int STAGE = (BM + BN) * kBK;
    __shared__ __attribute__((aligned(16))) bf16 smem[2 * STAGE];

    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    using ALoader = typename std::conditional<TA, RowContigLoader<BM>, KContigLoader<BM>>::type;
    using BLoader = typename std::conditional<TB, KContigLoader<BN>, RowContigLoader<BN>>::type;
    ALoader la;
    BLoader lb;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int nk = (p.K + kBK - 1) / kBK;
    la.load(p.A, p.lda, m0, p.M, 0, p.K);
    lb.load(p.B, p.ldb, n0, p.N, 0, p.K);
    la.store(smem);
    lb.store(smem + BM * kBK);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const bf16* As = smem + (kt & 1) * STAGE;
        const bf16* Bs = As + BM * kBK;
        if (kt + 1 < nk) {
            la.load(p.A, p.lda, m0, p.M, (kt + 1) * kBK, p.K);
            lb.load(p.B, p.ldb, n0, p.N, (kt + 1) * kBK, p.K);
        }
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int c = 2 * kk + (lane >> 5);
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int row = wm * WM + i * 32 + (lane & 31);
                af[i] = *reinterpret_cast<const bf16x8*>(As + row * kBK + ((c ^ swz(row)) << 3));
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int row = wn * WN + j * 32 + (lane & 31);
                bfr[j] = *reinterpret_cast<const bf16x8*>(Bs + row * kBK + ((c ^ swz(row)) << 3));
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            bf16* nxt = smem + ((kt + 1) & 1) * STAGE;
            la.store(nxt);
            lb.store(nxt + BM * kBK);
        }
        __syncthreads();
    }

    CT* C = static_cast<CT*>(p.C);
    const CT* R = static_cast<const CT*>(p.R);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = n0 + wn * WN + j * 32 + (lane & 31);
            if (n >= p.N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * WM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (m >= p.M) continue;
                float v = p.alpha * acc[i][j][e];
                const int64_t ci = static_cast<int64_t>(m) * p.ldc + n;
                if (p.beta != 0.0f) v += p.beta * ld(C, ci);
                if (R) v += ld(R, static_cast<int64_t>(m) * p.ldr + n);
                st(C, ci, v);
            }
        }
}

// ---------------------------------------------------------------------------------------
// Direct-to-LDS MFMA kernel.
// ---------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

__device__ __forceinline__ int swz_rc(int k) { return 4 * (k & 3); }

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt[3:0] in
// bits 3:0, expcnt 6:4, lgkmcnt 11:8, vmcnt[5:4] in 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Chunk swizzle of a K-contiguous [rows][BK] tile: the 16-byte chunk c of row r is stored
// at c ^ swz_kc(r), so the 16 rows read by one ds_read_b128 phase hit distinct banks.
template <int BK>
__device__ __forceinline__ int swz_kc(int r) {
    if constexpr (BK == 64) return (r ^ (r >> 3)) & 7;
    else return (r >> 2) & 3;  // BK == 32: four chunks per 64-byte row
}

// One wave's share of a ROWS x BK tile, copied HBM -> LDS with 1 KB per instruction.
// KC: K contiguous in HBM, LDS [ROWS][BK].  RC: rows contiguous in HBM, LDS [BK][ROWS].
template <int ROWS, int BK, bool KC>
__device__ __forceinline__ void dma_tile(const bf16* __restrict__ g, int64_t ld, int row0, int nrows, int k0, bf16* s) {
    constexpr int SEGS = ROWS * BK / 512;  // 512 bf16 = 1 KB per segment
    constexpr int PER_WAVE = SEGS / 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const int seg = wave * PER_WAVE + i;
        const bf16* src;
        if constexpr (KC) {
            constexpr int CPR = BK / 8;    // 16-byte chunks per row
            constexpr int RPS = 64 / CPR;  // rows per segment
            const int row = seg * RPS + lane / CPR;
            const int lc = (lane % CPR) ^ swz_kc<BK>(row);
            const int gr = min(row0 + row, nrows - 1);
            src = g + static_cast<int64_t>(gr) * ld + k0 + lc * 8;
        } else {
            constexpr int CPR = ROWS / 8;  // 16-byte chunks per k row
            constexpr int RPS = 64 / CPR;  // k rows per segment
            const int k = seg * RPS + lane / CPR;
            const int lc = (lane % CPR) ^ swz_rc(k);
            const int gr = min(row0 + lc * 8, nrows - 8);
            src = g + static_cast<int64_t>(k0 + k) * ld + gr;
        }
        dma16(src, s + seg * 512);
    }
}

// Instruction i (0 <= i < ROWS * BK / 2048) of this wave's share of a dma_tile copy.
template <int ROWS, int BK, bool KC>
__device__ __forceinline__ void dma_one(const bf16* __restrict__ g, int64_t ld, int row0, int nrows, int k0, bf16* s,
                                        int i) {
    constexpr int PER_WAVE = ROWS * BK / 512 / 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int seg = wave * PER_WAVE + i;
    const bf16* src;
    if constexpr (KC) {
        constexpr int CPR = BK / 8;
        constexpr int RPS = 64 / CPR;
        const int row = seg * RPS + lane / CPR;
        const int lc = (lane % CPR) ^ swz_kc<BK>(row);
        const int gr = min(row0 + row, nrows - 1);
        src = g + static_cast<int64_t>(gr) * ld + k0 + lc * 8;
    } else {
        constexpr int CPR = ROWS / 8;
        constexpr int RPS = 64 / CPR;
        const int k = seg * RPS + lane / CPR;
        const int lc = (lane % CPR) ^ swz_rc(k);
        const int gr = min(row0 + lc * 8, nrows - 8);
        src = g + static_cast<int64_t>(k0 + k) * ld + gr;
    }
    dma16(src, s + seg * 512);
}

// MFMA operand fragment (8 bf16 along k) for rows rb .. rb+31 of a tile, k step kk.
template <int ROWS, int BK, bool KC>
__device__ __forceinline__ bf16x8 frag(const bf16* t, int rb, int kk) {
    const int lane = threadIdx.x & 63;
    if constexpr (KC) {
        const int row = rb + (lane & 31);
        const int c = 2 * kk + (lane >> 5);
        return *reinterpret_cast<const bf16x8*>(t + row * BK + ((c ^ swz_kc<BK>(row)) << 3));
    } else {
        // ds_read_b64_tr_b16: within a group of 16 lanes, output lane i, slot j receives
        // element i % 4 of the 4 values addressed by source lane 4j + i / 4.  Source lane
        // s = 4j + q points at k row (kbase + j), columns m0 + 4q .. +3, so output lane i
        // holds column m0 + i for k rows kbase .. kbase+3.
        const int g = lane >> 4, s_ = lane & 15, j = s_ >> 2, q = s_ & 3;
        const int m = rb + 16 * (g & 1) + 4 * q;
        v4i16_t r[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = 16 * kk + 8 * (g >> 1) + 4 * h + j;
            const bf16* p = t + k * ROWS + (((m >> 3) ^ swz_rc(k)) << 3) + (m & 7);
            r[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p));
        }
        const uint2 a = __builtin_bit_cast(uint2, r[0]), b = __builtin_bit_cast(uint2, r[1]);
        return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
    }
}

// Wait until at most `tiles` later tiles' copies (LPT instructions each) are in flight.
template <int LPT>
__device__ __forceinline__ void wait_tiles(int tiles) {
    if (tiles >= 3) wait_vmcnt<3 * LPT>();
    else if (tiles == 2) wait_vmcnt<2 * LPT>();
    else if (tiles == 1) wait_vmcnt<LPT>();
    else wait_vmcnt<0>();
}

__device__ __forceinline__ void wait_lds() {
    // lgkmcnt(0), vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// Epilogue of the MFMA kernels: C = alpha * acc (+ beta * C) (+ R) for this block's tile.
// acc[i][j] holds the transposed 32x32 block (rows n, columns m) of wave (wm, wn).
template <int BM, int BN, int LDS_BYTES, typename CT>
__device__ __forceinline__ void gemm_epilogue(const MfmaParams& p, const f32x16 (&acc)[BM / 64][BN / 64], bf16* smem,
                                              int m0, int n0) {
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // Epilogue.  Lane owns output row m = mb + lane % 32 and, in block (i, j), the columns
    // n = nb + 8g + 4h + 0..3 (g = 0..3, h = lane / 32) in acc[i][j][4g .. 4g+3].
    CT* C = static_cast<CT*>(p.C);
    const CT* R = static_cast<const CT*>(p.R);
    const int h = lane >> 5;
    if (p.vec && m0 + BM <= p.M && n0 + BN <= p.N) {
        // Full tile: each wave stages its WM x WN sub-tile through its quarter of the (now
        // idle) LDS, so that every global store (and residual load) moves 16 contiguous
        // bytes per lane, whole rows per instruction.  After the loop's last barrier no wave
        // reads operand stages any more and no copy is in flight.
        constexpr int E = sizeof(CT);
        constexpr int RB = WN * E;                                       // bytes per sub-tile row
        constexpr int CPR = RB / 16;                                     // 16-byte chunks per row
        constexpr int REGION = LDS_BYTES / 4;  // LDS bytes per wave
        constexpr int FIT = REGION / RB < WM ? REGION / RB : WM;  // rows that fit the region
        constexpr int IB = FIT / 32;                                // 32-row blocks per pass
        constexpr int PASS_ROWS = IB * 32;                          // rows staged per pass
        constexpr int VE = 16 / E;     // elements per chunk
        constexpr int RPI = 64 / CPR;  // rows per 64-lane instruction
        static_assert(IB >= 1 && FM % IB == 0 && (CPR & (CPR - 1)) == 0 && PASS_ROWS % RPI == 0,
                      "epilogue staging");
        char* region = reinterpret_cast<char*>(smem) + wave * REGION;
        const int wrow0 = m0 + wm * WM, wcol0 = n0 + wn * WN;
#pragma unroll
        for (int i0 = 0; i0 < FM; i0 += IB) {
#pragma unroll
            for (int ii = 0; ii < IB; ++ii) {
                const int r = ii * 32 + (lane & 31);
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int byte = (32 * j + 8 * g + 4 * h) * E;
                        char* d = region + r * RB + (((byte >> 4) ^ (r & (CPR - 1))) << 4) + (byte & 15);
                        const f32x16& a = acc[i0 + ii][j];
                        const float v0 = p.alpha * a[4 * g], v1 = p.alpha * a[4 * g + 1];
                        const float v2 = p.alpha * a[4 * g + 2], v3 = p.alpha * a[4 * g + 3];
                        if constexpr (E == 2)
                            *reinterpret_cast<uint2*>(d) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
                        else
                            *reinterpret_cast<float4*>(d) = make_float4(v0, v1, v2, v3);
                    }
            }
            wait_lds();
#pragma unroll
            for (int t = 0; t < PASS_ROWS / RPI; ++t) {
                const int r = t * RPI + lane / CPR, c = lane % CPR;
                const uint4 raw = *reinterpret_cast<const uint4*>(region + r * RB + ((c ^ (r & (CPR - 1))) << 4));
                const int64_t gm = wrow0 + i0 * 32 + r;
                const int gn = wcol0 + c * VE;
                CT* dst = C + gm * p.ldc + gn;
                float v[VE];
                if constexpr (E == 2) {
                    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        v[2 * q] = __uint_as_float(w[q] << 16);
                        v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
                    }
                } else {
                    v[0] = __uint_as_float(raw.x); v[1] = __uint_as_float(raw.y);
                    v[2] = __uint_as_float(raw.z); v[3] = __uint_as_float(raw.w);
                }
                if (p.beta != 0.0f) {
#pragma unroll
                    for (int q = 0; q < VE; q += 4) {
                        float c4[4];
                        ld4(dst + q, c4);
#pragma unroll
                        for (int u = 0; u < 4; ++u) v[q + u] += p.beta * c4[u];
                    }
                }
                if (R) {
#pragma unroll
                    for (int q = 0; q < VE; q += 4) {
                        float r4[4];
                        ld4(R + gm * p.ldr + gn + q, r4);
#pragma unroll
                        for (int u = 0; u < 4; ++u) v[q + u] += r4[u];
                    }
                }
                if constexpr (E == 2) {
                    *reinterpret_cast<uint4*>(dst) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                                pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
                } else {
                    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
            wait_lds();  // the next pass overwrites the region
        }
        return;
    }
    const int nw = n0 + wn * WN + 4 * h;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm * WM + i * 32 + (lane & 31);
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int n = nw + j * 32 + 8 * (e >> 2) + (e & 3);
                if (n >= p.N) continue;
                float v = p.alpha * acc[i][j][e];
                const int64_t ci = static_cast<int64_t>(m) * p.ldc + n;
                if (p.beta != 0.0f) v += p.beta * ld(C, ci);
                if (R) v += ld(R, static_cast<int64_t>(m) * p.ldr + n);
                st(C, ci, v);
            }
    }
}

// acc += X2 Y2^T for this wave's 32x32 blocks: the low-rank term of a LoRA projection
// (forward: X2 = s x A^T, Y2 = B; backward: X2 = dxa, Y2 = A read k-major).  The operands are
// a few KB per tile, so fragments come straight from global memory (L2): 16 bytes per lane
// for rows contiguous in k, eight 2-byte loads (consecutive n across lanes) for a k-major Y2.
template <int FM, int FN, int WM, int WN>
__device__ __forceinline__ void rank_tail(const MfmaParams& p, f32x16 (&acc)[FM][FN], int m0, int n0, int wm,
                                          int wn) {
    const int lane = threadIdx.x & 63, hl = lane >> 5, r = lane & 31;
    const bf16* X2 = p.X2 + (p.seg_n > 0 ? static_cast<int64_t>(n0 / p.seg_n) * p.r2 : 0);
    const uint16_t* Y2 = reinterpret_cast<const uint16_t*>(p.Y2);
    for (int k0 = 0; k0 < p.r2; k0 += 16) {
        const int k = k0 + 8 * hl;
        const bool kin = k < p.r2;
        bf16x8 a[FM], b[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int m = m0 + wm * WM + i * 32 + r;
            const uint4 v = (kin && m < p.M) ? *reinterpret_cast<const uint4*>(X2 + static_cast<int64_t>(m) * p.ldx2 + k)
                                             : make_uint4(0, 0, 0, 0);
            a[i] = __builtin_bit_cast(bf16x8, v);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = n0 + wn * WN + j * 32 + r;
            const bool ok = kin && n < p.N;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (ok) {
                if (p.y2k) {
                    uint32_t w[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) w[q] = Y2[static_cast<int64_t>(k + q) * p.ldy2 + n];
                    v = make_uint4(w[0] | (w[1] << 16), w[2] | (w[3] << 16), w[4] | (w[5] << 16), w[6] | (w[7] << 16));
                } else {
                    v = *reinterpret_cast<const uint4*>(Y2 + static_cast<int64_t>(n) * p.ldy2 + k);
                }
            }
            b[j] = __builtin_bit_cast(bf16x8, v);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a[i], acc[i][j], 0, 0, 0);
    }
}

// Main loop schedule (per wave): fragments are double-buffered in registers; the reads of
// k step ks+1 are interleaved with the MFMAs of step ks (sched_group_barrier hints).  The
// barrier that publishes tile kt+1 sits before the MFMAs of the tile's last k step, so the
// MFMA pipe keeps working across it; right after it the freed stage receives tile kt+S and
// the first fragments of tile kt+1 are read while the last step's MFMAs issue.
template <int BM, int BN, int BK, int S, bool TA, bool TB, typename CT>
__device__ __forceinline__ void dma_body(const MfmaParams& p, int m0, int n0) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int KS = BK / 16;
    constexpr int STAGE = (BM + BN) * BK;
    constexpr bool AKC = !TA, BKC = TB;
    constexpr int LPT = (BM + BN) * BK / 512 / 4;  // copy instructions per wave per K step
    constexpr int NREAD = (AKC ? FM : 2 * FM) + (BKC ? FN : 2 * FN);  // LDS reads per k step
    constexpr int NMF = FM * FN;
    // the next step's fragment reads go out with the first half of this step's MFMAs, so
    // they have landed (no lgkmcnt stall) when the next step starts
    constexpr int HALF = NMF / 2 > 0 ? NMF / 2 : 1;
    constexpr int READS_PER_MF = (NREAD + HALF - 1) / HALF;
    constexpr int FRONT = (NREAD + READS_PER_MF - 1) / READS_PER_MF;  // MFMAs that carry reads
    static_assert(S >= 2 && S <= 5 && KS % 2 == 0, "stages / k steps");
    static_assert((S - 2) * LPT < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) bf16 smem[];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // split-K: this block's K range (k-contiguous operands move along columns, the others
    // along rows)
    const bf16* Ag = p.A;
    const bf16* Bg = p.B;
    if (blockIdx.y > 0) {
        const int64_t kz = static_cast<int64_t>(blockIdx.y) * p.K;
        Ag += AKC ? kz : kz * p.lda;
        Bg += BKC ? kz : kz * p.ldb;
    }

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    auto copy = [&](int tile, int stage) {
        bf16* dst = smem + stage * STAGE;
        dma_tile<BM, BK, AKC>(Ag, p.lda, m0, p.M, tile * BK, dst);
        dma_tile<BN, BK, BKC>(Bg, p.ldb, n0, p.N, tile * BK, dst + BM * BK);
    };
    auto read = [&](int stage, int kk, bf16x8* af, bf16x8* bfr) {
        const bf16* As = smem + stage * STAGE;
        const bf16* Bs = As + BM * BK;
#pragma unroll
        for (int i = 0; i < FM; ++i) af[i] = frag<BM, BK, AKC>(As, wm * WM + i * 32, kk);
#pragma unroll
        for (int j = 0; j < FN; ++j) bfr[j] = frag<BN, BK, BKC>(Bs, wn * WN + j * 32, kk);
    };
    constexpr int PA = BM * BK / 512 / 4;  // A-tile copy instructions per wave
    auto copy_one = [&](int tile, int stage, int q) {
        bf16* dst = smem + stage * STAGE;
        if (q < PA) dma_one<BM, BK, AKC>(Ag, p.lda, m0, p.M, tile * BK, dst, q);
        else dma_one<BN, BK, BKC>(Bg, p.ldb, n0, p.N, tile * BK, dst + BM * BK, q - PA);
    };
    auto read_one = [&](int stage, int kk, int f, bf16x8* af, bf16x8* bfr) {
        const bf16* As = smem + stage * STAGE;
        const bf16* Bs = As + BM * BK;
        if (f < FM) af[f] = frag<BM, BK, AKC>(As, wm * WM + f * 32, kk);
        else bfr[f - FM] = frag<BN, BK, BKC>(Bs, wn * WN + (f - FM) * 32, kk);
    };
    // B operand first: acc[i][j] accumulates the transposed 32x32 block (rows n, columns m),
    // so each lane ends up owning runs of four consecutive n of one output row m.
    auto mma = [&](const bf16x8* af, const bf16x8* bfr) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    };
    auto interleave = [&]() {
        // an MFMA leads each pair: no read is in flight ahead of the step's first MFMA,
        // whose operands were read a half step earlier
#pragma unroll
        for (int i = 0; i < FRONT; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);             // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, READS_PER_MF, 0);  // LDS reads
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NMF - FRONT, 0);  // the rest of the MFMAs
        __builtin_amdgcn_sched_barrier(0);  // nothing moves across k steps
    };

    const int nk = p.K / BK;
#pragma unroll
    for (int st = 0; st < S; ++st)
        if (st < nk) copy(st, st);
    wait_tiles<LPT>(min(S, nk) - 1);
    __builtin_amdgcn_s_barrier();
    bf16x8 fa[2][FM], fb[2][FN];
    read(0, 0, fa[0], fb[0]);
    // One K tile.  MC: tile kt+S exists (its copy goes into the freed stage); MT: tile kt+1
    // exists.  Both are compile-time, so the interleaved last k step has no branches.
    auto tile_step = [&](int kt, auto mc, auto mt) {
        constexpr bool MC = decltype(mc)::value, MT = decltype(mt)::value;
        const int cur = kt % S;
#pragma unroll
        for (int ks = 0; ks + 1 < KS; ++ks) {
            read(cur, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
            mma(fa[ks & 1], fb[ks & 1]);
            interleave();
        }
        wait_lds();  // this wave's reads of stage `cur` are complete
        // tile kt+1 has landed: at most min(S - 2, tiles after kt+1) later tiles in flight
        if constexpr (MC) wait_tiles<LPT>(S - 2);
        else if constexpr (MT) wait_tiles<LPT>(min(S - 2, nk - 1 - (kt + 1)));
        __builtin_amdgcn_s_barrier();
        // Last k step: its MFMAs, the copy of tile kt+S into the freed stage and the first
        // fragment reads of tile kt+1 go out interleaved one by one, so the copy issue never
        // holds back the MFMA pipe.
        const int nxt = (kt + 1) % S;
#pragma unroll
        for (int q = 0; q < NMF; ++q) {
            acc[q / FN][q % FN] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[1][q % FN], fa[1][q / FN], acc[q / FN][q % FN], 0, 0, 0);
            if constexpr (MC) {
#pragma unroll
                for (int c = q * LPT / NMF; c < (q + 1) * LPT / NMF; ++c) copy_one(kt + S, cur, c);
            }
            if constexpr (MT) {
                if (q < FM + FN) read_one(nxt, 0, q, fa[0], fb[0]);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the copies spread over the MFMAs
        }
    };
    using T1 = std::true_type;
    using F0 = std::false_type;
    int kt = 0;
    for (; kt + S < nk; ++kt) tile_step(kt, T1{}, T1{});
    for (; kt + 1 < nk; ++kt) tile_step(kt, F0{}, T1{});
    if (kt < nk) tile_step(kt, F0{}, F0{});

    if (p.r2 > 0) rank_tail<FM, FN, WM, WN>(p, acc, m0, n0, wm, wn);
    if (blockIdx.y > 0) {
        MfmaParams q = p;
        q.C = static_cast<float*>(p.C) + static_cast<int64_t>(blockIdx.y) * p.cz;
        gemm_epilogue<BM, BN, S * STAGE * 2, CT>(q, acc, smem, m0, n0);
    } else {
        gemm_epilogue<BM, BN, S * STAGE * 2, CT>(p, acc, smem, m0, n0);
    }
}

template <int BM, int BN, int BK, int S, bool TA, bool TB, typename CT>
__global__ __launch_bounds__(256, 1) void gemm_bf16_dma(const MfmaParams p) {
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    dma_body<BM, BN, BK, S, TA, TB, CT>(p, tm * BM, tn * BN);
}

// Grouped launch: the block's group, then its tile within the group.
template <int BM, int BN, int BK, int S, bool TA, bool TB, typename CT>
__global__ __launch_bounds__(256, 1) void gemm_bf16_dma_grouped(const DmaParams dp) {
    MfmaParams p = dp.p;
    const int bid = static_cast<int>(blockIdx.x);
    int g = 0;
    while (g + 1 < dp.ngroups && bid >= dp.g[g + 1].tile0) ++g;
    const GroupDesc& d = dp.g[g];
    p.A = d.A;
    p.B = d.B;
    p.C = d.C;
    p.lda = d.lda;
    p.ldb = d.ldb;
    p.ldc = d.ldc;
    p.M = d.M;
    p.N = d.N;
    p.K = d.K;
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    const int id = xcd_id(bid - d.tile0, d.nblocks);
    if (id >= tiles_m * tiles_n) return;  // a group's padding block (the whole block leaves)
    int tm, tn;
    id_to_tile(id, tiles_m, tiles_n, tm, tn);
    dma_body<BM, BN, BK, S, TA, TB, CT>(p, tm * BM, tn * BN);
}

// C = alpha * sum_z P[z] + beta * C + R over the split-K partials P [splits][M][N] (fp32,
// summed in z order: deterministic).
template <typename CT>
__global__ __launch_bounds__(256) void splitk_reduce_k(const float* __restrict__ P, int splits, int64_t pz, int M, int N,
                                                       float alpha, float beta, CT* C, int64_t ldc, const CT* R,
                                                       int64_t ldr) {
    const int64_t total = static_cast<int64_t>(M) * N;
    for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int m = static_cast<int>(i / N), n = static_cast<int>(i % N);
        float acc = P[i];
        for (int z = 1; z < splits; ++z) acc += P[z * pz + i];
        const int64_t ci = static_cast<int64_t>(m) * ldc + n;
        float v = alpha * acc;
        if (beta != 0.0f) v += beta * ld(C, ci);
        if (R) v += ld(R, static_cast<int64_t>(m) * ldr + n);
        st(C, ci, v);
    }
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int BM, int BN, bool TA, bool TB, typename CT>
void launch_mfma(const GemmArgs& a, hipStream_t s) {
    MfmaParams p;
    p.A = static_cast<const bf16*>(a.A);
    p.B = static_cast<const bf16*>(a.B);
    p.C = a.C;
    p.R = a.R;
    p.lda = a.lda; p.ldb = a.ldb; p.ldc = a.ldc; p.ldr = a.ldr;
    p.M = static_cast<int>(a.M); p.N = static_cast<int>(a.N); p.K = static_cast<int>(a.K);
    p.alpha = a.alpha; p.beta = a.beta;
    p.vec = 0;
    p.X2 = p.Y2 = nullptr;
    p.ldx2 = p.ldy2 = p.cz = 0;
    p.r2 = p.seg_n = p.y2k = 0;
    const int tiles = static_cast<int>(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    hipLaunchKernelGGL((gemm_bf16_mfma<BM, BN, TA, TB, CT>), dim3(tiles), dim3(256), 0, s, p);
    AIC_LAUNCH_CHECK("gemm_bf16_mfma");
}

// splits > 1: the K range is cut into `splits` equal parts (K % (64 splits) == 0), block z
// writes its fp32 partial to part + z M N, and splitk_reduce_k forms C.  Otherwise the
// low-rank term of `a` (if any) runs in the kernel's tail.
template <int BM, int BN, int BK, int S, bool TA, bool TB, typename CT>
void launch_dma(const GemmArgs& a, hipStream_t s, int splits = 1, float* part = nullptr) {
    MfmaParams p;
    p.A = static_cast<const bf16*>(a.A);
    p.B = static_cast<const bf16*>(a.B);
    p.C = a.C;
    p.R = a.R;
    p.lda = a.lda; p.ldb = a.ldb; p.ldc = a.ldc; p.ldr = a.ldr;
    p.M = static_cast<int>(a.M); p.N = static_cast<int>(a.N); p.K = static_cast<int>(a.K);
    p.alpha = a.alpha; p.beta = a.beta;
    p.X2 = static_cast<const bf16*>(a.X2);
    p.Y2 = static_cast<const bf16*>(a.Y2);
    p.ldx2 = a.ldx2; p.ldy2 = a.ldy2;
    p.r2 = static_cast<int>(a.r2); p.seg_n = static_cast<int>(a.seg_n); p.y2k = a.y2_kmajor;
    p.cz = 0;
    if (splits > 1) {
        p.C = part;
        p.R = nullptr;
        p.ldc = a.N;
        p.ldr = 0;
        p.alpha = 1.0f;
        p.beta = 0.0f;
        p.K = static_cast<int>(a.K / splits);
        p.cz = a.M * a.N;
        p.r2 = 0;
    }
    p.vec = p.ldc % 4 == 0 && aligned16(p.C) && (!p.R || (p.ldr % 4 == 0 && aligned16(p.R)));
    const int tiles = static_cast<int>(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    constexpr size_t lds = static_cast<size_t>(S) * (BM + BN) * BK * sizeof(uint16_t);
    static_assert(lds <= 160 * 1024, "LDS per block");
    static bool configured = false;  // one attribute call per instantiation
    if (!configured) {
        AIC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_bf16_dma<BM, BN, BK, S, TA, TB, CT>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        configured = true;
    }
    hipLaunchKernelGGL((gemm_bf16_dma<BM, BN, BK, S, TA, TB, CT>), dim3(tiles, splits), dim3(256), lds, s, p);
    AIC_LAUNCH_CHECK("gemm_bf16_dma");
}

// One launch for several products of the same shape class (see DmaParams).
template <int BM, int BN, int BK, int S, bool TA, bool TB, typename CT>
void launch_dma_grouped(const GemmArgs* a, int n, hipStream_t s) {
    DmaParams dp;
    MfmaParams& p = dp.p;
    p.A = static_cast<const bf16*>(a[0].A);
    p.B = static_cast<const bf16*>(a[0].B);
    p.C = a[0].C;
    p.R = nullptr;
    p.lda = a[0].lda; p.ldb = a[0].ldb; p.ldc = a[0].ldc; p.ldr = 0;
    p.M = static_cast<int>(a[0].M); p.N = static_cast<int>(a[0].N); p.K = static_cast<int>(a[0].K);
    p.alpha = a[0].alpha; p.beta = a[0].beta;
    p.X2 = p.Y2 = nullptr;
    p.ldx2 = p.ldy2 = p.cz = 0;
    p.r2 = p.seg_n = p.y2k = 0;
    p.vec = 1;
    dp.ngroups = n;
    int blocks = 0;
    for (int i = 0; i < n; ++i) {
        const int tiles = static_cast<int>(((a[i].M + BM - 1) / BM) * ((a[i].N + BN - 1) / BN));
        GroupDesc& d = dp.g[i];
        d.A = static_cast<const bf16*>(a[i].A);
        d.B = static_cast<const bf16*>(a[i].B);
        d.C = a[i].C;
        d.lda = a[i].lda; d.ldb = a[i].ldb; d.ldc = a[i].ldc;
        d.M = static_cast<int>(a[i].M); d.N = static_cast<int>(a[i].N); d.K = static_cast<int>(a[i].K);
        d.tile0 = blocks;
        d.nblocks = (tiles + 7) / 8 * 8;
        blocks += d.nblocks;
        p.vec = p.vec && a[i].ldc % 4 == 0 && aligned16(a[i].C);
    }
    for (int i = n; i < kMaxGroups; ++i) dp.g[i] = dp.g[0];
    constexpr size_t lds = static_cast<size_t>(S) * (BM + BN) * BK * sizeof(uint16_t);
    static bool configured = false;
    if (!configured) {
        AIC_HIP_CHECK(hipFuncSetAttribute(
            reinterpret_cast<const void*>(&gemm_bf16_dma_grouped<BM, BN, BK, S, TA, TB, CT>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        configured = true;
    }
    hipLaunchKernelGGL((gemm_bf16_dma_grouped<BM, BN, BK, S, TA, TB, CT>), dim3(blocks), dim3(256), lds, s, dp);
    AIC_LAUNCH_CHECK("gemm_bf16_dma_grouped");
}

template <int BM, int BN, int BK, int S, typename CT>
void dispatch_grouped(const GemmArgs* a, int n, hipStream_t s) {
    if (!a[0].transA && a[0].transB) launch_dma_grouped<BM, BN, BK, S, false, true, CT>(a, n, s);
    else if (!a[0].transA && !a[0].transB) launch_dma_grouped<BM, BN, BK, S, false, false, CT>(a, n, s);
    else if (a[0].transA && !a[0].transB) launch_dma_grouped<BM, BN, BK, S, true, false, CT>(a, n, s);
    else launch_dma_grouped<BM, BN, BK, S, true, true, CT>(a, n, s);
}

template <int BM, int BN, int BK, int S, typename CT>
void dispatch_dma(const GemmArgs& a, hipStream_t s, int splits = 1, float* part = nullptr) {
    if (!a.transA && a.transB) launch_dma<BM, BN, BK, S, false, true, CT>(a, s, splits, part);
    else if (!a.transA && !a.transB) launch_dma<BM, BN, BK, S, false, false, CT>(a, s, splits, part);
    else if (a.transA && !a.transB) launch_dma<BM, BN, BK, S, true, false, CT>(a, s, splits, part);
    else launch_dma<BM, BN, BK, S, true, true, CT>(a, s, splits, part);
}

template <int BM, int BN, typename CT>
void dispatch_trans(const GemmArgs& a, hipStream_t s) {
    if (!a.transA && a.transB) launch_mfma<BM, BN, false, true, CT>(a, s);
    else if (!a.transA && !a.transB) launch_mfma<BM, BN, false, false, CT>(a, s);
    else if (a.transA && !a.transB) launch_mfma<BM, BN, true, false, CT>(a, s);
    else launch_mfma<BM, BN, true, true, CT>(a, s);
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

bool gemm_dma_eligible(const GemmArgs& a) {
    if (!gemm_mfma_eligible(a)) return false;
    if (a.K % 64 || a.M < 8 || a.N < 8) return false;
    return true;
}

namespace {

// C = alpha * (sum of the split-K partials) + beta * C + R.
void splitk_reduce(const float* part, int splits, const GemmArgs& a, hipStream_t s) {
    const int64_t total = a.M * a.N;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 4096));
    if (a.c == DType::Float32)
        hipLaunchKernelGGL(splitk_reduce_k<float>, dim3(grid), dim3(256), 0, s, part, splits, total,
                           static_cast<int>(a.M), static_cast<int>(a.N), a.alpha, a.beta, static_cast<float*>(a.C),
                           a.ldc, static_cast<const float*>(a.R), a.ldr);
    else
        hipLaunchKernelGGL(splitk_reduce_k<bf16>, dim3(grid), dim3(256), 0, s, part, splits, total,
                           static_cast<int>(a.M), static_cast<int>(a.N), a.alpha, a.beta, static_cast<bf16*>(a.C),
                           a.ldc, static_cast<const bf16*>(a.R), a.ldr);
    AIC_LAUNCH_CHECK("splitk_reduce_k");
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

void gemm(const GemmArgs& a, hipStream_t s) {
    AIC_CHECK(a.M >= 0 && a.N >= 0 && a.K >= 0, InvalidArgument, "negative GEMM size");
    AIC_CHECK(a.M < (1LL << 31) && a.N < (1LL << 31) && a.K < (1LL << 31), InvalidArgument, "GEMM size too large");
    AIC_CHECK(a.A && a.B && a.C, InvalidArgument, "null GEMM operand");
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
    if (gemm_dma_eligible(a)) {
        // 256x256 tiles from half a round of tiles up (measured on the 1B shapes: 176 tiles of
        // 256x256 beat 704 of 128x128 by 24%); between 32 and 128 of them over a long K, 256x256
        // tiles with K split so that about one full round runs (the 2048x2048x8192 weight
        // gradient: 80 us against 93 us on 128x128 tiles)
        const int64_t t256 = ((a.M + 255) / 256) * ((a.N + 255) / 256);
        const int64_t t128 = ((a.M + 127) / 128) * ((a.N + 127) / 128);
        const bool big = t256 >= 128;
        int splits256 = 1;
        if (a.r2 == 0 && !big && t256 >= 32 && a.K >= 4096) {
            splits256 = static_cast<int>(std::min<int64_t>(4, 256 / t256));
            while (splits256 > 1 && a.K % (64LL * splits256)) --splits256;
        }
        if (a.r2 > 0) {
            const int64_t bn = big ? 256 : 128;
            const bool tail = a.r2 % 8 == 0 && a.ldx2 % 8 == 0 && aligned16(a.X2) &&
                              (a.y2_kmajor || (a.ldy2 % 8 == 0 && aligned16(a.Y2))) &&
                              (a.seg_n == 0 || a.seg_n % bn == 0);
            if (!tail) {
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
    bool one_launch = n >= 2 && n <= kMaxGroups;
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
        for (int i = 0; i < n; ++i) gemm(a[i], s);
        return;
    }
    if (a[0].c == DType::Float32) {
        if (t256 >= 128) dispatch_grouped<256, 256, 64, 2, float>(a, n, s);
        else dispatch_grouped<128, 128, 64, 4, float>(a, n, s);
    } else {
        if (t256 >= 128) dispatch_grouped<256, 256, 64, 2, bf16>(a, n, s);
        else dispatch_grouped<128, 128, 64, 4, bf16>(a, n, s);
    }
}

}  // namespace aic::hip
