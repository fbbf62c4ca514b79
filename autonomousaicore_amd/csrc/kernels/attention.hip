// Causal flash attention forward/backward.
//
// Replaces launch_flash_attention_forward/backward_gpu (src/cuda/cuda_flash_attention.cu,
// one 64-thread block per query row, fp32, wrong for head_dim > 64) and the default
// materialised path of CausalSelfAttention (include/nn/attention.hpp:84-119).  Same
// mathematics: softmax(Q K^T * scale + causal mask) V with the row log-sum-exp saved.
//
// bf16 path (head_dim 64 / 128), v_mfma_f32_32x32x16_bf16, wave64:
//   * Q/K/V/dO tiles travel HBM -> LDS with global_load_lds_dwordx4 (no register staging)
//     into [rows][head_dim] tiles whose 16-byte chunks are XOR-swizzled per row.  Row
//     operands are read with ds_read_b128; transposed operands (V^T, K^T, Q^T, dO^T) are read
//     from the same tiles with ds_read_b64_tr_b16, so no transposed copy is kept.
//   * forward  one block = 128 queries (4 waves x 32).  A wave computes S^T = K Q^T so a
//              lane owns one query: the row max/sum need one exchange with lane ^ 32 and the
//              rescale of the output accumulator O^T is per lane.  P^T feeds
//              O^T += V^T P^T from the accumulator registers (the MFMA k order is permuted
//              identically on the V^T side).  Masking runs only on diagonal tiles; the scale
//              is folded into one FMA before exp2; O is rescaled only when a row max grows by
//              more than 2^8 (values stay below 2^8 otherwise, exactly as rescaling would).
//              Software-pipelined: the scores of tile t+1 are computed while tile t's
//              exponentials run, and P(t) V(t) while tile t+1's row max runs.
//   * backward two kernels, no atomics (deterministic):
//              dK/dV: one block = 128 keys (4 waves x 32) over 64-query tiles; S and dP are
//              [query x key] so a lane owns a key and P / dS feed dV^T += dO^T P and
//              dK^T += Q^T dS from registers.
//              dQ:   one block = 128 queries over 64-key tiles (dQ^T += K^T dS^T).
// fp32 path (the fp32 reference configuration, head_dim 16/32/64/128): SIMT kernels, fp32 math.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazyRescale = 8.0f;  // log2 units

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

// ---------------------------------------------------------------------------------------
// [rows][HD] bf16 tiles in LDS, 16-byte chunks XOR-swizzled per row.  The swizzle depends
// on row % 16 only and makes both read patterns bank-conflict free: a ds_read_b128 phase
// (16 consecutive rows, one logical chunk) touches 16 distinct bank slots, and each half of
// a ds_read_b64_tr_b16 (4 consecutive rows x 64 bytes) covers the banks exactly once.
// ---------------------------------------------------------------------------------------
template <int HD>
__device__ __forceinline__ int swz(int row) {
    if constexpr (HD == 128) return 4 * (row & 3) | ((row >> 2) & 3);
    else return 4 * ((row >> 1) & 1) | ((row >> 2) & 3);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

// This wave's quarter of a 64 x HD tile: rows [row0, row0 + 64) of a [tokens][ld] matrix
// (head offset applied by the caller), rows >= nrows clamped (their values are never used).
template <int HD>
__device__ __forceinline__ void dma_rows64(const bf16* __restrict__ g, int64_t ld, int row0, int nrows, bf16* s) {
    constexpr int NC = HD / 8, RPS = 64 / NC;  // chunks per row, rows per 1 KB segment
    constexpr int PER_WAVE = 64 * HD / 512 / 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const int seg = wave * PER_WAVE + i;
        const int row = seg * RPS + lane / NC;
        const int lc = (lane % NC) ^ swz<HD>(row);
        const int gr = min(row0 + row, nrows - 1);
        dma16(g + static_cast<int64_t>(gr) * ld + lc * 8, s + seg * 512);
    }
}

// The same copies with the address split into a wave-uniform base (the tile's first row, in
// SGPRs) and per-lane 32-bit byte offsets computed once per kernel, so a tile's copy costs no
// per-lane address arithmetic; a tile reaching past nrows takes dma_rows64 (per-lane clamping).
// Offsets stay below 2^32 for leading dimensions under 2^24 (mfma_ok).
template <int HD>
struct Rows64 {
    static constexpr int NC = HD / 8, RPS = 64 / NC, PER_WAVE = 64 * HD / 512 / 4;
    uint32_t voff[PER_WAVE];
    int seg0;
    __device__ __forceinline__ void init(int64_t ld) {
        const int lane = threadIdx.x & 63;
        seg0 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * PER_WAVE;
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
            const int row = (seg0 + i) * RPS + lane / NC;
            const int lc = (lane % NC) ^ swz<HD>(row);
            voff[i] = static_cast<uint32_t>(2 * (static_cast<int64_t>(row) * ld + lc * 8));
        }
    }
    __device__ __forceinline__ void copy(const bf16* __restrict__ g, int64_t ld, int row0, int nrows, bf16* s) const {
        if (row0 + 64 > nrows) {
            dma_rows64<HD>(g, ld, row0, nrows, s);
            return;
        }
        const bf16* base = g + static_cast<int64_t>(row0) * ld;
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) dma16s(base, voff[i], s + (seg0 + i) * 512);
    }
};

// MFMA operand fragments of a swizzled [rows][HD] tile, addressed through per-lane byte
// offsets computed once per kernel (every read is then a register base plus an immediate).
//   row(t, rb, kk): lane = row rb + lane%32 (rb a multiple of 32), 8 values of k step kk
//                   along head_dim (ds_read_b128).
//   tr(t, ob, ks):  lane = head_dim column 32ob + lane%32, 8 values along rows in the
//                   permuted order of a 16-row step ks (elements 0..3: rows 16ks + 4h + 0..3,
//                   elements 4..7: rows 16ks + 8 + 4h + 0..3, h = lane / 32), read with two
//                   ds_read_b64_tr_b16: within a group of 16 lanes, output lane i slot j takes
//                   element i % 4 of the 4 values at source lane 4j + i / 4, so source lane
//                   s = 4j + q addresses row (base + j), columns cb' + 4q .. +3.
template <int HD>
struct Frags {
    static constexpr int KS = HD / 16, OB = HD / 32, RB = HD * 2;  // RB: bytes per row
    int row_off[KS];
    int tr_off[OB][2];
    __device__ __forceinline__ void init() {
        const int lane = threadIdx.x & 63;
        const int h = lane >> 5, r = lane & 31;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) row_off[kk] = r * RB + (((2 * kk + h) ^ swz<HD>(r)) << 4);
        const int g = lane >> 4, s = lane & 15, j = s >> 2, q = s & 3;
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int row = 8 * u + 4 * h + j;
                const int col = 32 * ob + 16 * (g & 1) + 4 * q;
                tr_off[ob][u] = row * RB + (((col >> 3) ^ swz<HD>(row)) << 4) + (col & 7) * 2;
            }
    }
    __device__ __forceinline__ bf16x8 row(const char* t, int rb, int kk) const {
        return *reinterpret_cast<const bf16x8*>(t + rb * RB + row_off[kk]);
    }
    __device__ __forceinline__ bf16x8 tr(const char* t, int ob, int ks) const {
        const v4i16_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(t + 16 * ks * RB + tr_off[ob][0]));
        const v4i16_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(t + 16 * ks * RB + tr_off[ob][1]));
        const uint2 x = __builtin_bit_cast(uint2, a), y = __builtin_bit_cast(uint2, b);
        return __builtin_bit_cast(bf16x8, make_uint4(x.x, x.y, y.x, y.y));
    }
};

__device__ __forceinline__ bf16x8 pack_bf16x8(const f32x16& a, int off) {
    return __builtin_bit_cast(bf16x8, make_uint4(pack_bf16x2(a[off], a[off + 1]), pack_bf16x2(a[off + 2], a[off + 3]),
                                                 pack_bf16x2(a[off + 4], a[off + 5]),
                                                 pack_bf16x2(a[off + 6], a[off + 7])));
}

__device__ __forceinline__ uint4 ldg16(const bf16* p, bool ok) {
    return ok ? *reinterpret_cast<const uint4*>(p) : make_uint4(0, 0, 0, 0);
}

__device__ __forceinline__ void zero(f32x16& a) {
#pragma unroll
    for (int e = 0; e < 16; ++e) a[e] = 0.0f;
}

// Writes a [32 rows of head_dim] x [lane = token] accumulator block as token rows.
__device__ __forceinline__ void store_t(bf16* row_ptr, const f32x16& acc, int ob, float mul) {
    const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int d0 = ob * 32 + 8 * g + 4 * h;
        *reinterpret_cast<uint2*>(row_ptr + d0) =
            make_uint2(pack_bf16x2(acc[4 * g] * mul, acc[4 * g + 1] * mul),
                       pack_bf16x2(acc[4 * g + 2] * mul, acc[4 * g + 3] * mul));
    }
}

// ---------------------------------------------------------------------------------------
// Forward
// store_t of a whole [head_dim] x [lane = token] accumulator with the adjoint of the half-split
// rotary embedding applied on the way out (RoPEBackward, include/nn/rope.hpp:23-112, as rope_k
// with INV): for d < head_dim / 2, with a1 = mul acc[d] and a2 = mul acc[d + head_dim / 2],
// out[d] = a1 cos + a2 sin and out[d + head_dim / 2] = a2 cos - a1 sin, where cos / sin are the
// token's table rows.  The partner of row d sits in block ob + OB / 2 of the same lane.
template <int OB>
__device__ __forceinline__ void store_rot(bf16* row_ptr, const f32x16 (&acc)[OB], float mul, const float* cos_row,
                                          const float* sin_row) {
    constexpr int HALF = OB * 16;
    const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int ob = 0; ob < OB / 2; ++ob)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = ob * 32 + 8 * g + 4 * h;
            const float4 c4 = *reinterpret_cast<const float4*>(cos_row + d0);
            const float4 s4 = *reinterpret_cast<const float4*>(sin_row + d0);
            const float cc[4] = {c4.x, c4.y, c4.z, c4.w}, ss[4] = {s4.x, s4.y, s4.z, s4.w};
            float o1[4], o2[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float a1 = acc[ob][4 * g + u] * mul, a2 = acc[ob + OB / 2][4 * g + u] * mul;
                o1[u] = a1 * cc[u] + a2 * ss[u];
                o2[u] = a2 * cc[u] - a1 * ss[u];
            }
            *reinterpret_cast<uint2*>(row_ptr + d0) = make_uint2(pack_bf16x2(o1[0], o1[1]), pack_bf16x2(o1[2], o1[3]));
            *reinterpret_cast<uint2*>(row_ptr + HALF + d0) =
                make_uint2(pack_bf16x2(o2[0], o2[1]), pack_bf16x2(o2[2], o2[3]));
        }
}

// ---------------------------------------------------------------------------------------
// Forward, software-pipelined.  Copy unit t holds K of tile t+1 and V of tile t, so while a wave
// multiplies P(t) V(t) it already holds the scores of tile t+1.  Per iteration two MFMA groups,
// each pinned in source order (sched_barrier after every MFMA) with the work that overlaps it:
//   A  S(t+1) = K(t+1) Q^T (2 KS MFMAs) + the exponentials, row sum and bf16 packing of tile t,
//      the K fragment reads two steps ahead and the first V^T reads of group B
//   B  O^T += V(t)^T P(t)^T (4 OB MFMAs) + the (masked) row max of tile t+1 while it moves into
//      the current-tile registers, and the V^T reads one step ahead
// then the lazy-rescale decision for tile t+1 (a wave-uniform branch, rarely taken) and one
// barrier, after which unit t+2 goes into the stage unit t used.  Per query the arithmetic and
// its order are those of the unpipelined tile loop (scores, max, rescale, exponentials, row sum,
// P V; measured bit-identical to it, and 8% faster at the 1B shape); a wave's fully masked tiles
// (causal diagonal) are multiplied with P = 0 instead of skipped, so the four waves keep one
// schedule.
template <int HD>
__global__ __launch_bounds__(256, 2) void attn_fwd_pipe(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                        const bf16* __restrict__ v, int64_t ldq, bf16* __restrict__ o,
                                                        int64_t ldo, float* __restrict__ lse, int H, int S, float c,
                                                        int causal) {
    constexpr int BQ = 128, BKV = 64, KS = HD / 16, OB = HD / 32, TILE = BKV * HD;
    constexpr int NA = 2 * KS;     // MFMAs of group A
    constexpr int NB = 4 * OB;     // MFMAs of group B
    constexpr int EA = 32 / NA;    // exponentials per group A slot
    constexpr int EB = 32 / NB;    // row-max elements per group B slot
    constexpr int NR = OB + 1;     // V^T fragment ring
    constexpr int KR = 3;          // K fragment ring (reads two MFMAs ahead; deeper measured no faster)
    static_assert(32 % NA == 0 && 32 % NB == 0 && NA >= OB, "slot counts");
    __shared__ __attribute__((aligned(16))) bf16 sm[2][2 * TILE];  // per stage: K(t+1), V(t)

    const int nq = (S + BQ - 1) / BQ;
    const int BH = static_cast<int>(gridDim.x) / nq;
    const int qb = nq - 1 - static_cast<int>(blockIdx.x) / BH;
    const int bh = static_cast<int>(blockIdx.x) % BH, h = bh % H, b = bh / H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
    const int q0 = qb * BQ, qw = q0 + wave * 32, myq = qw + (lane & 31);
    const int64_t tok0 = static_cast<int64_t>(b) * S, hoff = static_cast<int64_t>(h) * HD;
    const bf16* kb = k + tok0 * ldq + hoff;
    const bf16* vb = v + tok0 * ldq + hoff;

    bf16x8 qf[KS];
    {
        const bf16* qp = q + (tok0 + myq) * ldq + hoff + 8 * hl;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) qf[kk] = __builtin_bit_cast(bf16x8, ldg16(qp + 16 * kk, myq < S));
    }
    Frags<HD> F;
    F.init();
    f32x16 oacc[OB];
#pragma unroll
    for (int i = 0; i < OB; ++i) zero(oacc[i]);
    float m_run = -INFINITY, l_run = 0.0f;

    const int kv_end = causal ? min(S, q0 + BQ) : S;
    const int nt = (kv_end + BKV - 1) / BKV;  // >= 1
    // tiles from `mask0` on hold keys past some query of the block (causal) or past S
    const int mask0 = min(causal ? q0 / BKV : nt, S / BKV);
    // head_dim 64: per-lane addressing (measured 2% faster there)
    [[maybe_unused]] Rows64<HD> rows;
    if constexpr (HD == 128) rows.init(ldq);
    auto copy_rows = [&](const bf16* g, int t, bf16* dst) {
        if constexpr (HD == 128) rows.copy(g, ldq, t * BKV, S, dst);
        else dma_rows64<HD>(g, ldq, t * BKV, S, dst);
    };
    auto copy_k = [&](int t, int st) { copy_rows(kb, t, sm[st]); };
    auto unit = [&](int t, int st) {
        if (t + 1 < nt) copy_k(t + 1, st);
        copy_rows(vb, t, sm[st] + TILE);
    };
    // element e of key block jb is key k0 + 32 jb + 8 (e >> 2) + 4 hl + (e & 3)
    auto masked = [&](int k0, int jb, int e) {
        const int key = k0 + jb * 32 + 8 * (e >> 2) + 4 * hl + (e & 3);
        return (causal && key > myq) || key >= S;
    };
    // the row max of a tile's scores -> the reference max and the rescale of O and l
    auto absorb = [&](float mx) {
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const bool grow = (mx - m_run) * c > kLazyRescale;
        if (__any(grow)) {
            const float m_new = grow ? mx : m_run;
            const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_new) * c);
            l_run *= alpha;
#pragma unroll
            for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[ob][e] *= alpha;
            m_run = m_new;
        }
    };

    f32x16 sc[2], sn[2];  // scores of the current tile t and of tile t+1
    copy_k(0, 0);
    unit(0, 1);
    if (nt > 1) wait_vmcnt<2 * (64 * HD / 512 / 4)>();  // K(0) has landed; unit 0 may be in flight
    else wait_vmcnt<64 * HD / 512 / 4>();
    __builtin_amdgcn_s_barrier();
    {
        const char* Kb = reinterpret_cast<const char*>(sm[0]);
        zero(sc[0]);
        zero(sc[1]);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
                sc[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.row(Kb, jb * 32, kk), qf[kk], sc[jb], 0, 0, 0);
        if (mask0 == 0)
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (masked(0, jb, e)) sc[jb][e] = -INFINITY;
        float mx = sc[0][0];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sc[jb][e]);
        absorb(mx);
    }
    wait_lds();
    wait_vmcnt<0>();  // unit 0
    __builtin_amdgcn_s_barrier();
    if (1 < nt) unit(1, 0);

    // One iteration.  HN: tile t+1 exists; MK: it needs the mask.
    auto iter = [&](int t, auto hn, auto mk) {
        constexpr bool HN = decltype(hn)::value, MK = decltype(mk)::value;
        const int st = (t + 1) & 1;
        const char* Kb = reinterpret_cast<const char*>(sm[st]);
        const char* Vb = reinterpret_cast<const char*>(sm[st] + TILE);
        const float moff = -m_run * c;
        bf16x8 rk[KR], tv[NR], pf[4];
        auto rd_k = [&](int g) { rk[g % KR] = F.row(Kb, 32 * (g / KS), g % KS); };
        auto rd_v = [&](int f) { tv[f % NR] = F.tr(Vb, f % OB, f / OB); };
        float rs = 0.0f;
        if constexpr (HN) {
            zero(sn[0]);
            zero(sn[1]);
#pragma unroll
            for (int g = 0; g < KR - 1; ++g) rd_k(g);
        }
        // A
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            if constexpr (HN) {
                const int jb = i / KS, kk = i % KS;
                sn[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rk[i % KR], qf[kk], sn[jb], 0, 0, 0);
                if (i + KR - 1 < NA) rd_k(i + KR - 1);
            }
#pragma unroll
            for (int x = i * EA; x < (i + 1) * EA; ++x) {
                const int jb = x >> 4, e = x & 15;
                const float p = __builtin_amdgcn_exp2f(fmaf(sc[jb][e], c, moff));
                sc[jb][e] = p;
                rs += p;
                if ((e & 7) == 7) pf[2 * jb + (e >> 3)] = pack_bf16x8(sc[jb], e - 7);
            }
            if (i >= NA - OB) rd_v(i - (NA - OB));
            if constexpr (HN) __builtin_amdgcn_sched_barrier(0);
        }
        rs += __shfl_xor(rs, 32, 64);
        l_run += rs;
        // B
        const int k1 = (t + 1) * BKV;
        float mx = -INFINITY;
#pragma unroll
        for (int f = 0; f < NB; ++f) {
            const int ks = f / OB, ob = f % OB;
            oacc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tv[f % NR], pf[ks], oacc[ob], 0, 0, 0);
            if (f + OB < NB) rd_v(f + OB);
            if constexpr (HN) {
#pragma unroll
                for (int x = f * EB; x < (f + 1) * EB; ++x) {
                    const int jb = x >> 4, e = x & 15;
                    float s = sn[jb][e];
                    if constexpr (MK) s = masked(k1, jb, e) ? -INFINITY : s;
                    sc[jb][e] = s;
                    mx = fmaxf(mx, s);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (HN) absorb(mx);
        wait_lds();
        wait_vmcnt<0>();  // unit t+1
        __builtin_amdgcn_s_barrier();  // every wave is done with unit t's stage; unit t+1 is visible
        if (t + 2 < nt) unit(t + 2, st);
    };
    using T1 = std::true_type;
    using F0 = std::false_type;
    int t = 0;
    for (; t + 1 < nt && t + 1 < mask0; ++t) iter(t, T1{}, F0{});
    for (; t + 1 < nt; ++t) iter(t, T1{}, T1{});
    iter(t, F0{}, F0{});

    if (myq < S) {
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
        bf16* op = o + (tok0 + myq) * ldo + hoff;
#pragma unroll
        for (int ob = 0; ob < OB; ++ob) store_t(op, oacc[ob], ob, inv);
        if (hl == 0) lse[(static_cast<int64_t>(b) * H + h) * S + myq] = (m_run * c + log2f(l_run)) * kLn2;
    }
}

// D[b,h,s] = sum_d dO * O  (fp32), one wave per (token, head).
template <typename T>
__global__ __launch_bounds__(256) void attn_dot_k(const T* __restrict__ o, const T* __restrict__ dout, int64_t ldo,
                                                  float* __restrict__ D, int64_t Ttok, int H, int S, int HD) {
    const int64_t gw = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (gw >= Ttok * H) return;
    const int64_t t = gw / H;
    const int h = static_cast<int>(gw % H);
    float acc = 0.0f;
    for (int d = lane; d < HD; d += 64) {
        const int64_t i = t * ldo + static_cast<int64_t>(h) * HD + d;
        acc += ld(o, i) * ld(dout, i);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        const int64_t b = t / S, s = t % S;
        D[(b * H + h) * S + s] = acc;
    }
}

// The same for bf16 rows of HD % 8 == 0 elements with 16-byte loads: HD / 8 lanes per
// (token, head) row, 64 / (HD / 8) rows per wave; each lane's eight products, then a
// butterfly over the row's lanes.
template <int HD>
__global__ __launch_bounds__(256) void attn_dot_v8_k(const bf16* __restrict__ o, const bf16* __restrict__ dout,
                                                     int64_t ldo, float* __restrict__ D, int64_t Ttok, int H, int S) {
    constexpr int LPR = HD / 8, RPW = 64 / LPR;
    const int64_t gw = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63, sub = lane % LPR;
    const int64_t row = gw * RPW + lane / LPR;
    const bool ok = row < Ttok * H;
    float acc = 0.0f;
    if (ok) {
        const int64_t t = row / H;
        const int h = static_cast<int>(row % H);
        const int64_t i = t * ldo + static_cast<int64_t>(h) * HD + sub * 8;
        const uint4 a = *reinterpret_cast<const uint4*>(o + i), b = *reinterpret_cast<const uint4*>(dout + i);
        const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc += __uint_as_float(wa[q] << 16) * __uint_as_float(wb[q] << 16);
            acc += __uint_as_float(wa[q] & 0xffff0000u) * __uint_as_float(wb[q] & 0xffff0000u);
        }
    }
#pragma unroll
    for (int w = LPR / 2; w > 0; w >>= 1) acc += __shfl_xor(acc, w);
    if (ok && sub == 0) {
        const int64_t t = row / H, b = t / S, s = t % S;
        const int h = static_cast<int>(row % H);
        D[(b * H + h) * S + s] = acc;
    }
}

// ---------------------------------------------------------------------------------------
// Backward: dK, dV.  Stage = Q tile, dO tile (64 x HD each), lse and D of the 64 queries.
//
// Per query tile a wave (32 keys) runs four groups of MFMAs, each pinned in source order
// (sched_barrier after every MFMA) together with the work that overlaps it:
//   A  S^T, dP^T of queries 0..31   (2 KS MFMAs) + fragment reads two k steps ahead
//   B  S^T, dP^T of queries 32..63  (2 KS)      + the softmax / dS of queries 0..31, one
//                                                 element per slot, and the transposed reads
//                                                 of the first dV / dK step
//   C  dV^T, dK^T over queries 0..31 (4 OB)     + the softmax / dS of queries 32..63 and the
//                                                 transposed reads one step ahead
//   D  dV^T, dK^T over queries 32..63 (4 OB)    + the transposed reads one step ahead
// so the LDS latency of every fragment and the softmax VALU run in the shadow of MFMAs.  The
// causal mask is one compare per element against a per-lane bound (no branch).
// head_dim 128 (about 500 registers: one block per CU): three stages, the copy of tile t+2 going
// out right after the barrier that opens tile t, into the stage tile t-1 used, so one barrier per
// tile suffices.  head_dim 64: two stages and two blocks per CU (the other block's waves hide
// what the schedule does not; measured faster than three stages at one block).
// ---------------------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256, HD == 128 ? 1 : 2) void attn_bwd_dkdv_mfma(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int64_t ldq,
    const bf16* __restrict__ dout, int64_t ldo, const float* __restrict__ lse, const float* __restrict__ Dg,
    bf16* __restrict__ dk, bf16* __restrict__ dv, int64_t ldd, int H, int S, float c, float scale, int causal,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin) {
    constexpr int BQ = 64, BKV = 128, KS = HD / 16, OB = HD / 32, TILE = BQ * HD;
    constexpr int LPT = 2 * (64 * HD / 512 / 4);
    constexpr int NST = HD == 128 ? 3 : 2;
    constexpr int STAGE = 2 * TILE + 2 * 64 * 2;  // Q, dO, then lse and D as fp32 (2 x 64 x 4 B)
    constexpr int NA = 2 * KS;                    // MFMAs of groups A and B
    constexpr int NC = 2 * OB * 2;                // MFMAs of groups C and D (two 16-query steps)
    constexpr int EB = 16 / NA;                   // softmax elements per slot in group B
    constexpr int EC = 16 / NC;                   // ... in group C
    static_assert(16 % NA == 0 && 16 % NC == 0, "slot counts");
    __shared__ __attribute__((aligned(16))) bf16 sm[NST][STAGE];

    // 1-D grid, heaviest blocks first (causal: key block 0 sees every query tile)
    const int nkv = (S + BKV - 1) / BKV;
    const int BH = static_cast<int>(gridDim.x) / nkv;
    const int kblk = static_cast<int>(blockIdx.x) / BH;
    const int bh = static_cast<int>(blockIdx.x) % BH, h = bh % H, b = bh / H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
    const int k0 = kblk * BKV, kw = k0 + wave * 32, mykey = kw + (lane & 31);
    const int64_t tok0 = static_cast<int64_t>(b) * S, hoff = static_cast<int64_t>(h) * HD;
    const float* lse_bh = lse + (static_cast<int64_t>(b) * H + h) * S;
    const float* D_bh = Dg + (static_cast<int64_t>(b) * H + h) * S;

    bf16x8 kf[KS], vf[KS];
    {
        const bf16* kp = k + (tok0 + mykey) * ldq + hoff + 8 * hl;
        const bf16* vp = v + (tok0 + mykey) * ldq + hoff + 8 * hl;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            kf[kk] = __builtin_bit_cast(bf16x8, ldg16(kp + 16 * kk, mykey < S));
            vf[kk] = __builtin_bit_cast(bf16x8, ldg16(vp + 16 * kk, mykey < S));
        }
    }
    Frags<HD> F;
    F.init();
    f32x16 dvt[OB], dkt[OB];
#pragma unroll
    for (int i = 0; i < OB; ++i) {
        zero(dvt[i]);
        zero(dkt[i]);
    }

    const int nq = (S + BQ - 1) / BQ;
    const int qt0 = causal ? (k0 / BQ) : 0;
    // waves 0 and 1 also copy the 64 lse / D values of the tile (4 bytes per lane); rows past S
    // repeat row S-1 (their lse is replaced by +inf below, so they contribute nothing)
    // head_dim 64 keeps the per-lane addressing: its two blocks per CU leave no registers for
    // the offsets
    [[maybe_unused]] Rows64<HD> rows_q, rows_o;
    if constexpr (HD == 128) {
        rows_q.init(ldq);
        rows_o.init(ldo);
    }
    auto copy = [&](int qt, int st) {
        if constexpr (HD == 128) {
            rows_q.copy(q + tok0 * ldq + hoff, ldq, qt * BQ, S, sm[st]);
            rows_o.copy(dout + tok0 * ldo + hoff, ldo, qt * BQ, S, sm[st] + TILE);
        } else {
            dma_rows64<HD>(q + tok0 * ldq + hoff, ldq, qt * BQ, S, sm[st]);
            dma_rows64<HD>(dout + tok0 * ldo + hoff, ldo, qt * BQ, S, sm[st] + TILE);
        }
        if (wave < 2) {
            const float* src = (wave == 0 ? lse_bh : D_bh) + min(qt * BQ + lane, S - 1);
            dma4(src, sm[st] + 2 * TILE + wave * 128);
        }
    };
    if (qt0 < nq) copy(qt0, 0);
    if (qt0 + 1 < nq) copy(qt0 + 1, 1);

    for (int qt = qt0; qt < nq; ++qt) {
        const int it = qt - qt0, st = it % NST;
        // tile qt has landed (tile qt+1's copy may still be in flight) and every wave is done
        // with tile qt-1, whose stage receives tile qt+2
        if (qt + 1 < nq) {
            if (wave < 2) wait_vmcnt<LPT + 1>();
            else wait_vmcnt<LPT>();
        } else {
            wait_vmcnt<0>();
        }
        wait_lds();  // this wave's reads of tile qt-1's stage are complete
        __builtin_amdgcn_s_barrier();
        if (NST == 3 && qt + 2 < nq) copy(qt + 2, (it + 2) % NST);
        const int qs = qt * BQ;
        // every query of the tile precedes this wave's keys: nothing to do
        // EDGE: the tile holds queries before some key of this wave (causal) or past S, so the
        // mask and the past-S rows are applied; other tiles skip those selects (wave-uniform)
        const bool tail = qs + BQ > S;
        const bool edge = (causal && qs < kw + 31) || tail;
        auto work = [&](auto edge_c) {
        constexpr bool EDGE = decltype(edge_c)::value;
        const char* Qb = reinterpret_cast<const char*>(sm[st]);
        const char* Ob = reinterpret_cast<const char*>(sm[st] + TILE);
        const float* Ls = reinterpret_cast<const float*>(sm[st] + 2 * TILE);
        const float* Ds = Ls + 64;
        // element e of query block jb is query qs + 32 jb + 8 (e >> 2) + 4 hl + (e & 3): masked
        // when its offset 32 jb + 8 (e >> 2) + (e & 3) is below lo (causal: key > query)
        const int lo = causal ? mykey - qs - 4 * hl : -(1 << 30);

        f32x16 sa[2], sd[2];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            zero(sa[jb]);
            zero(sd[jb]);
        }
        bf16x8 rq[3], ro[3];  // row fragments, g = jb * KS + kk in slot g % 3
        auto rd = [&](int g) {
            rq[g % 3] = F.row(Qb, 32 * (g / KS), g % KS);
            ro[g % 3] = F.row(Ob, 32 * (g / KS), g % KS);
        };
        // -lse * log2(e) and D of element group G = 4 jb + (e >> 2) (its four queries), in rings
        // of three float4: read from LDS two groups ahead, lse scaled one group ahead (queries
        // past S: -inf, so p = exp2(-inf) = 0), so they hold 24 registers instead of 64
        float4 lr[3], dr[3];
        auto rd_q = [&](int G) {
            const int qi = 32 * (G >> 2) + 8 * (G & 3) + 4 * hl;
            lr[G % 3] = *reinterpret_cast<const float4*>(Ls + qi);
            dr[G % 3] = *reinterpret_cast<const float4*>(Ds + qi);
        };
        auto scale_l = [&](int G) {
            const int qi = 32 * (G >> 2) + 8 * (G & 3) + 4 * hl;
            float4& l = lr[G % 3];
            float v[4] = {l.x, l.y, l.z, l.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if constexpr (EDGE) v[u] = qs + qi + u >= S ? -INFINITY : -v[u] * kLog2e;
                else v[u] = -v[u] * kLog2e;
            }
            l = make_float4(v[0], v[1], v[2], v[3]);
        };
        auto comp = [](const float4& f, int u) { return u == 0 ? f.x : u == 1 ? f.y : u == 2 ? f.z : f.w; };
        // The softmax of element e in two stages a slot apart, so the exponential's latency
        // passes under the next MFMA instead of holding up its issue: sm1 takes the exponential,
        // sm2 (the next slot) the mask, P and dS.
        float pe[2][16];
        auto sm1 = [&](int jb, int e) {
            const int G = 4 * jb + (e >> 2);
            if ((e & 3) == 0) {
                if (G + 2 < 8) rd_q(G + 2);
                if (G + 1 < 8) scale_l(G + 1);
            }
            pe[jb][e] = __builtin_amdgcn_exp2f(fmaf(sa[jb][e], c, comp(lr[G % 3], e & 3)));
        };
        auto sm2 = [&](int jb, int e) {
            const int G = 4 * jb + (e >> 2);
            float p = pe[jb][e];
            if constexpr (EDGE) p = (32 * jb + 8 * (e >> 2) + (e & 3) < lo) ? 0.0f : p;
            sa[jb][e] = p;
            sd[jb][e] = p * (sd[jb][e] - comp(dr[G % 3], e & 3));
        };
        bf16x8 pf[4], dsf[4];
        auto pack = [&](int ks) {
            pf[ks] = pack_bf16x8(sa[ks >> 1], 8 * (ks & 1));
            dsf[ks] = pack_bf16x8(sd[ks >> 1], 8 * (ks & 1));
        };
        // transposed fragments f = ks * 2 OB + i (i < OB: dO^T block i, else Q^T block i - OB) of
        // the four 16-query steps, read one step ahead into a ring of 2 OB + 1
        constexpr int NR = 2 * OB + 1;
        bf16x8 tr[NR];
        auto rd_tr = [&](int f) {
            const int ks = f / (2 * OB), i = f % (2 * OB);
            tr[f % NR] = i < OB ? F.tr(Ob, i, ks) : F.tr(Qb, i - OB, ks);
        };

        rd(0);
        rd(1);
        rd_q(0);
        rd_q(1);
        // A: S^T, dP^T of queries 0..31
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int kk = i >> 1, g = kk;
            if ((i & 1) == 0) {
                sa[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rq[g % 3], kf[kk], sa[0], 0, 0, 0);
                rd(g + 2);
            } else {
                sd[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ro[g % 3], vf[kk], sd[0], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        scale_l(0);
        // B: S^T, dP^T of queries 32..63; softmax of queries 0..31; transposed reads of step 0
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int kk = i >> 1, g = KS + kk;
            if ((i & 1) == 0) {
                sa[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rq[g % 3], kf[kk], sa[1], 0, 0, 0);
                if (g + 2 < 2 * KS) rd(g + 2);
            } else {
                sd[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ro[g % 3], vf[kk], sd[1], 0, 0, 0);
            }
            if (i > 0) {  // the second stage of the previous slot's elements
#pragma unroll
                for (int e = (i - 1) * EB; e < i * EB; ++e) sm2(0, e);
                if (i * EB == 8) pack(0);
            }
#pragma unroll
            for (int e = i * EB; e < (i + 1) * EB; ++e) sm1(0, e);
            if (i < 2 * OB) rd_tr(i);
            __builtin_amdgcn_sched_barrier(0);
        }
        // C, D: dV^T += dO^T P, dK^T += Q^T dS over the four 16-query steps
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
            for (int i = 0; i < 2 * OB; ++i) {
                const int f = ks * 2 * OB + i;
                if (i < OB)
                    dvt[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr[f % NR], pf[ks], dvt[i], 0, 0, 0);
                else
                    dkt[i - OB] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr[f % NR], dsf[ks], dkt[i - OB], 0, 0, 0);
                if (f + 2 * OB < 8 * OB) rd_tr(f + 2 * OB);
                if (f == 0) {  // the last slot of group B, second stage
#pragma unroll
                    for (int e = (NA - 1) * EB; e < NA * EB; ++e) sm2(0, e);
                    pack(1);
                }
                if (ks < 2 || f == 4 * OB) {  // group C: the softmax of queries 32..63
                    const int slot = ks * 2 * OB + i;
                    if (slot > 0) {
#pragma unroll
                        for (int e = (slot - 1) * EC; e < slot * EC; ++e) sm2(1, e);
                        if (slot * EC == 8) pack(2);
                        if (slot * EC == 16) pack(3);
                    }
                    if (ks < 2) {
#pragma unroll
                        for (int e = slot * EC; e < (slot + 1) * EC; ++e) sm1(1, e);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        };
        if (!causal || qs + BQ - 1 >= kw) {
            if (edge) work(std::true_type{});
            else work(std::false_type{});
        }
        if constexpr (NST == 2) {  // every wave is done with stage st before tile qt+2 lands there
            wait_lds();
            __builtin_amdgcn_s_barrier();
            if (qt + 2 < nq) copy(qt + 2, st);
        }
    }

    if (mykey < S) {
        bf16* dkp = dk + (tok0 + mykey) * ldd + hoff;
        bf16* dvp = dv + (tok0 + mykey) * ldd + hoff;
        if (rope_cos) {  // dK leaves with the rotary embedding's adjoint applied
            store_rot<OB>(dkp, dkt, scale, rope_cos + static_cast<int64_t>(mykey) * (HD / 2),
                          rope_sin + static_cast<int64_t>(mykey) * (HD / 2));
        } else {
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) store_t(dkp, dkt[ob], ob, scale);
        }
#pragma unroll
        for (int ob = 0; ob < OB; ++ob) store_t(dvp, dvt[ob], ob, 1.0f);
    }
}

// ---------------------------------------------------------------------------------------
// Backward: dQ.  Stage = K tile, V tile.
// ---------------------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_mfma(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                           const bf16* __restrict__ v, int64_t ldq,
                                                           const bf16* __restrict__ o, const bf16* __restrict__ dout,
                                                           int64_t ldo, const float* __restrict__ lse,
                                                           float* __restrict__ Dg, bf16* __restrict__ dq, int64_t ldd,
                                                           int H, int S, float c, float scale, int causal,
                                                           const float* __restrict__ rope_cos,
                                                           const float* __restrict__ rope_sin) {
    constexpr int BQ = 128, BKV = 64, KS = HD / 16, OB = HD / 32, TILE = BKV * HD;
    constexpr int LPT = 2 * (64 * HD / 512 / 4);
    __shared__ __attribute__((aligned(16))) bf16 sm[2][2 * TILE];

    // 1-D grid, heaviest blocks first over all (batch, head) pairs: block id -> (tile, bh)
    const int nq = (S + BQ - 1) / BQ;
    const int BH = static_cast<int>(gridDim.x) / nq;
    const int qb = nq - 1 - static_cast<int>(blockIdx.x) / BH;
    const int bh = static_cast<int>(blockIdx.x) % BH, h = bh % H, b = bh / H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
    const int q0 = qb * BQ, qw = q0 + wave * 32, myq = qw + (lane & 31);
    const int64_t tok0 = static_cast<int64_t>(b) * S, hoff = static_cast<int64_t>(h) * HD;

    bf16x8 qf[KS], df[KS];
    {
        const bf16* qp = q + (tok0 + myq) * ldq + hoff + 8 * hl;
        const bf16* dp_ = dout + (tok0 + myq) * ldo + hoff + 8 * hl;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            qf[kk] = __builtin_bit_cast(bf16x8, ldg16(qp + 16 * kk, myq < S));
            df[kk] = __builtin_bit_cast(bf16x8, ldg16(dp_ + 16 * kk, myq < S));
        }
    }
    const float my_l2 = myq < S ? lse[(static_cast<int64_t>(b) * H + h) * S + myq] * kLog2e : 0.0f;
    // D = sum over head_dim of dO * O (fp32) for this lane's query: the lane's half of the row
    // (the chunks its dO fragments hold), then the other half from lane ^ 32.  Written out for
    // the dK/dV kernel, which runs after this one.
    float my_D;
    {
        const bf16* op = o + (tok0 + myq) * ldo + hoff + 8 * hl;
        float part = 0.0f;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            const uint4 ov = ldg16(op + 16 * kk, myq < S);
            const uint4 dv = __builtin_bit_cast(uint4, df[kk]);
            const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w}, dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                part = fmaf(__uint_as_float(dw[i] << 16), __uint_as_float(ow[i] << 16), part);
                part = fmaf(__uint_as_float(dw[i] & 0xffff0000u), __uint_as_float(ow[i] & 0xffff0000u), part);
            }
        }
        my_D = part + __shfl_xor(part, 32, 64);
        if (hl == 0 && myq < S) Dg[(static_cast<int64_t>(b) * H + h) * S + myq] = my_D;
    }
    Frags<HD> F;
    F.init();
    f32x16 dqt[OB];
#pragma unroll
    for (int i = 0; i < OB; ++i) zero(dqt[i]);

    const int kv_end = causal ? min(S, q0 + BQ) : S;
    const int ntiles = (kv_end + BKV - 1) / BKV;
    Rows64<HD> rows;
    rows.init(ldq);
    auto copy = [&](int t, int st) {
        rows.copy(k + tok0 * ldq + hoff, ldq, t * BKV, S, sm[st]);
        rows.copy(v + tok0 * ldq + hoff, ldq, t * BKV, S, sm[st] + TILE);
    };
    if (ntiles > 0) copy(0, 0);
    if (ntiles > 1) copy(1, 1);

    // one K/V tile (stc: its stage when known at compile time, else -1)
    auto tile = [&](int t, auto stc) {
        constexpr int ST0 = decltype(stc)::value;
        const int st = ST0 >= 0 ? ST0 : (t & 1);
        if (t + 1 < ntiles) wait_vmcnt<LPT>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        const int k0 = t * BKV;
        const char* Kb = reinterpret_cast<const char*>(sm[st]);
        const char* Vb = reinterpret_cast<const char*>(sm[st] + TILE);
        if (!causal || k0 <= qw + 31) {
            f32x16 s[2], dp[2];
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) {
                zero(s[jb]);
                zero(dp[jb]);
            }
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
#pragma unroll
                for (int jb = 0; jb < 2; ++jb) {
                    s[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.row(Kb, jb * 32, kk), qf[kk], s[jb], 0, 0,
                                                                     0);
                    dp[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.row(Vb, jb * 32, kk), df[kk], dp[jb], 0,
                                                                      0, 0);
                }
            // wave-uniform: the tile holds keys past some query of the wave (causal) or past S.
            // Queries past S need no mask: their q, dO, lse and D are 0, so dS = 1 * (0 - 0) = 0.
            // Only such tiles run the compare and select: their masked scores become -inf, whose
            // exp2 below is 0 exactly as a select of 0 would be.
            const bool diag = (causal && k0 + BKV - 1 > qw) || k0 + BKV > S;
            if (diag) {
                // element (jb, e) is key k0 + 32 jb + 8 (e >> 2) + 4 hl + (e & 3): masked when its
                // offset 32 jb + 8 (e >> 2) + (e & 3) exceeds lim
                const int lim = min(causal ? myq : S - 1, S - 1) - k0 - 4 * hl;
#pragma unroll
                for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        if (32 * jb + 8 * (e >> 2) + (e & 3) > lim) s[jb][e] = -INFINITY;
            }
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[jb][e], c, -my_l2));
                    dp[jb][e] = p * (dp[jb][e] - my_D);
                }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 dsf = pack_bf16x8(dp[ks >> 1], 8 * (ks & 1));
#pragma unroll
                for (int ob = 0; ob < OB; ++ob)
                    dqt[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.tr(Kb, ob, ks), dsf, dqt[ob], 0, 0,
                                                                       0);
            }
        }
        wait_lds();
        __builtin_amdgcn_s_barrier();
        if (t + 2 < ntiles) copy(t + 2, st);
    };
    // (a loop over stage pairs, with the stage a compile-time constant, spills here)
    for (int t = 0; t < ntiles; ++t) tile(t, std::integral_constant<int, -1>{});

    if (myq < S) {
        bf16* dqp = dq + (tok0 + myq) * ldd + hoff;
        if (rope_cos) {  // dQ leaves with the rotary embedding's adjoint applied
            store_rot<OB>(dqp, dqt, scale, rope_cos + static_cast<int64_t>(myq) * (HD / 2),
                          rope_sin + static_cast<int64_t>(myq) * (HD / 2));
        } else {
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) store_t(dqp, dqt[ob], ob, scale);
        }
    }
}

// ---------------------------------------------------------------------------------------
// SIMT path (fp32 configuration, any dtype, head_dim 16/32/64/128): one thread per query row
// (forward, dQ) or key row (dK, dV); fp32 math; K/V or Q/dO tiles staged in LDS.
// ---------------------------------------------------------------------------------------
constexpr int kSimtTile = 64;

template <typename T, int HD>
__global__ __launch_bounds__(64) void attn_fwd_simt(const T* __restrict__ q, const T* __restrict__ k,
                                                    const T* __restrict__ v, int64_t ldq, int64_t ldk,
                                                    T* __restrict__ o, int64_t ldo, float* __restrict__ lse, int H,
                                                    int S, int Sk, float scale, int causal) {
    __shared__ float sk[kSimtTile][HD + 1];
    __shared__ float sv[kSimtTile][HD + 1];
    const int h = blockIdx.y, b = blockIdx.z;
    const int qi = blockIdx.x * kSimtTile + threadIdx.x;
    const int64_t tok0 = static_cast<int64_t>(b) * S, tok0k = static_cast<int64_t>(b) * Sk;
    const int64_t hoff = static_cast<int64_t>(h) * HD;
    float qv[HD], acc[HD];
    for (int d = 0; d < HD; ++d) {
        qv[d] = qi < S ? ld(q, (tok0 + qi) * ldq + hoff + d) : 0.0f;
        acc[d] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    const int kend = causal ? min(Sk, static_cast<int>((blockIdx.x + 1) * kSimtTile)) : Sk;
    for (int k0 = 0; k0 < kend; k0 += kSimtTile) {
        __syncthreads();
        for (int e = threadIdx.x; e < kSimtTile * HD; e += 64) {
            const int r = e / HD, d = e % HD;
            const int key = k0 + r;
            sk[r][d] = key < Sk ? ld(k, (tok0k + key) * ldk + hoff + d) : 0.0f;
            sv[r][d] = key < Sk ? ld(v, (tok0k + key) * ldk + hoff + d) : 0.0f;
        }
        __syncthreads();
        if (qi >= S) continue;
        for (int r = 0; r < kSimtTile; ++r) {
            const int key = k0 + r;
            if (key >= Sk || (causal && key > qi)) break;
            float sdot = 0.0f;
            for (int d = 0; d < HD; ++d) sdot += qv[d] * sk[r][d];
            const float x = sdot * scale;
            const float mn = fmaxf(m, x);
            const float a = expf(m - mn);
            const float p = expf(x - mn);
            l = l * a + p;
            for (int d = 0; d < HD; ++d) acc[d] = acc[d] * a + p * sv[r][d];
            m = mn;
        }
    }
    if (qi < S) {
        for (int d = 0; d < HD; ++d) st(o, (tok0 + qi) * ldo + hoff + d, acc[d] / l);
        lse[(static_cast<int64_t>(b) * H + h) * S + qi] = m + logf(l);
    }
}

// dK, dV: one thread per key; loops over queries >= key.
template <typename T, int HD>
__global__ __launch_bounds__(64) void attn_bwd_kv_simt(const T* __restrict__ q, const T* __restrict__ k,
                                                       const T* __restrict__ v, int64_t ldq, int64_t ldk,
                                                       const T* __restrict__ dout, int64_t ldo,
                                                       const float* __restrict__ lse, const float* __restrict__ Dg,
                                                       T* dk, T* dv, int64_t ldd, int64_t lddk, int H, int S, int Sk,
                                                       float scale, int causal) {
    __shared__ float sq[kSimtTile][HD + 1];
    __shared__ float sdo[kSimtTile][HD + 1];
    __shared__ float sl[kSimtTile], sD[kSimtTile];
    const int h = blockIdx.y, b = blockIdx.z;
    const int kj = blockIdx.x * kSimtTile + threadIdx.x;
    const int64_t tok0 = static_cast<int64_t>(b) * S, tok0k = static_cast<int64_t>(b) * Sk;
    const int64_t hoff = static_cast<int64_t>(h) * HD;
    const float* lse_bh = lse + (static_cast<int64_t>(b) * H + h) * S;
    const float* D_bh = Dg + (static_cast<int64_t>(b) * H + h) * S;
    float kv_[HD], vv[HD], dka[HD], dva[HD];
    for (int d = 0; d < HD; ++d) {
        kv_[d] = kj < Sk ? ld(k, (tok0k + kj) * ldk + hoff + d) : 0.0f;
        vv[d] = kj < Sk ? ld(v, (tok0k + kj) * ldk + hoff + d) : 0.0f;
        dka[d] = 0.0f;
        dva[d] = 0.0f;
    }
    const int qstart = causal ? static_cast<int>(blockIdx.x * kSimtTile) : 0;
    for (int q0 = qstart; q0 < S; q0 += kSimtTile) {
        __syncthreads();
        for (int e = threadIdx.x; e < kSimtTile * HD; e += 64) {
            const int r = e / HD, d = e % HD;
            const int qq = q0 + r;
            sq[r][d] = qq < S ? ld(q, (tok0 + qq) * ldq + hoff + d) : 0.0f;
            sdo[r][d] = qq < S ? ld(dout, (tok0 + qq) * ldo + hoff + d) : 0.0f;
        }
        if (threadIdx.x < kSimtTile) {
            const int qq = q0 + threadIdx.x;
            sl[threadIdx.x] = qq < S ? lse_bh[qq] : 0.0f;
            sD[threadIdx.x] = qq < S ? D_bh[qq] : 0.0f;
        }
        __syncthreads();
        if (kj >= Sk) continue;
        for (int r = 0; r < kSimtTile; ++r) {
            const int qq = q0 + r;
            if (qq >= S) break;
            if (causal && kj > qq) continue;
            float sdot = 0.0f, dpd = 0.0f;
            for (int d = 0; d < HD; ++d) {
                sdot += sq[r][d] * kv_[d];
                dpd += sdo[r][d] * vv[d];
            }
            const float p = expf(sdot * scale - sl[r]);
            const float ds = p * (dpd - sD[r]);
            for (int d = 0; d < HD; ++d) {
                dva[d] += p * sdo[r][d];
                dka[d] += ds * sq[r][d];
            }
        }
    }
    if (kj < Sk)
        for (int d = 0; d < HD; ++d) {
            st(dk, (tok0k + kj) * lddk + hoff + d, dka[d] * scale);
            st(dv, (tok0k + kj) * lddk + hoff + d, dva[d]);
        }
}

template <typename T, int HD>
__global__ __launch_bounds__(64) void attn_bwd_q_simt(const T* __restrict__ q, const T* __restrict__ k,
                                                      const T* __restrict__ v, int64_t ldq, int64_t ldk,
                                                      const T* __restrict__ dout, int64_t ldo,
                                                      const float* __restrict__ lse, const float* __restrict__ Dg, T* dq,
                                                      int64_t ldd, int H, int S, int Sk, float scale, int causal) {
    __shared__ float sk[kSimtTile][HD + 1];
    __shared__ float sv[kSimtTile][HD + 1];
    const int h = blockIdx.y, b = blockIdx.z;
    const int qi = blockIdx.x * kSimtTile + threadIdx.x;
    const int64_t tok0 = static_cast<int64_t>(b) * S, tok0k = static_cast<int64_t>(b) * Sk;
    const int64_t hoff = static_cast<int64_t>(h) * HD;
    float qv[HD], dov[HD], acc[HD];
    for (int d = 0; d < HD; ++d) {
        qv[d] = qi < S ? ld(q, (tok0 + qi) * ldq + hoff + d) : 0.0f;
        dov[d] = qi < S ? ld(dout, (tok0 + qi) * ldo + hoff + d) : 0.0f;
        acc[d] = 0.0f;
    }
    const float l = qi < S ? lse[(static_cast<int64_t>(b) * H + h) * S + qi] : 0.0f;
    const float Dq = qi < S ? Dg[(static_cast<int64_t>(b) * H + h) * S + qi] : 0.0f;
    const int kend = causal ? min(Sk, static_cast<int>((blockIdx.x + 1) * kSimtTile)) : Sk;
    for (int k0 = 0; k0 < kend; k0 += kSimtTile) {
        __syncthreads();
        for (int e = threadIdx.x; e < kSimtTile * HD; e += 64) {
            const int r = e / HD, d = e % HD;
            const int key = k0 + r;
            sk[r][d] = key < Sk ? ld(k, (tok0k + key) * ldk + hoff + d) : 0.0f;
            sv[r][d] = key < Sk ? ld(v, (tok0k + key) * ldk + hoff + d) : 0.0f;
        }
        __syncthreads();
        if (qi >= S) continue;
        for (int r = 0; r < kSimtTile; ++r) {
            const int key = k0 + r;
            if (key >= Sk || (causal && key > qi)) break;
            float sdot = 0.0f, dpd = 0.0f;
            for (int d = 0; d < HD; ++d) {
                sdot += qv[d] * sk[r][d];
                dpd += dov[d] * sv[r][d];
            }
            const float p = expf(sdot * scale - l);
            const float ds = p * (dpd - Dq);
            for (int d = 0; d < HD; ++d) acc[d] += ds * sk[r][d];
        }
    }
    if (qi < S)
        for (int d = 0; d < HD; ++d) st(dq, (tok0 + qi) * ldd + hoff + d, acc[d] * scale);
}

// ---------------------------------------------------------------------------------------
// Attention over a KV cache (decode): block (i, h, b) is query i of the S_new new tokens at
// position start_pos + i; it attends to cache rows 0 .. start_pos + i.  Scores go to LDS
// (one wave per key, lanes across head_dim, shuffle sums), then max, exp and sum in fixed
// trees, then each thread accumulates one head_dim column over a strided key subset and the
// subsets are added in a fixed order.  fp32 math; the row sums are deterministic.
// ---------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void attn_cached_k(const T* __restrict__ q, int64_t ldq, const T* __restrict__ kc,
                                                     const T* __restrict__ vc, int64_t ldkv, int64_t bstride,
                                                     T* __restrict__ o, int64_t ldo, int S_new, int start_pos, int hd,
                                                     float scale) {
    extern __shared__ float sm_dec[];
    const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int L = start_pos + i + 1;
    float* sc = sm_dec;           // [L] scores, then probabilities
    float* red = sm_dec + L;      // [256]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const T* qr = q + (static_cast<int64_t>(b) * S_new + i) * ldq + static_cast<int64_t>(h) * hd;
    const T* kb = kc + static_cast<int64_t>(b) * bstride + static_cast<int64_t>(h) * hd;
    const T* vb = vc + static_cast<int64_t>(b) * bstride + static_cast<int64_t>(h) * hd;
    const float q0 = lane < hd ? ld(qr, lane) : 0.0f, q1 = lane + 64 < hd ? ld(qr, lane + 64) : 0.0f;
    for (int j = wave; j < L; j += 4) {
        const T* kr = kb + static_cast<int64_t>(j) * ldkv;
        float p = (lane < hd ? q0 * ld(kr, lane) : 0.0f) + (lane + 64 < hd ? q1 * ld(kr, lane + 64) : 0.0f);
#pragma unroll
        for (int w = 32; w > 0; w >>= 1) p += __shfl_xor(p, w);
        if (lane == 0) sc[j] = p * scale;
    }
    __syncthreads();
    float m = -INFINITY;
    for (int j = tid; j < L; j += 256) m = fmaxf(m, sc[j]);
    red[tid] = m;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) red[tid] = fmaxf(red[tid], red[tid + w]);
        __syncthreads();
    }
    m = red[0];
    __syncthreads();
    float sum = 0.0f;
    for (int j = tid; j < L; j += 256) {
        const float e = expf(sc[j] - m);
        sc[j] = e;
        sum += e;
    }
    red[tid] = sum;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) red[tid] += red[tid + w];
        __syncthreads();
    }
    const float inv = 1.0f / red[0];
    __syncthreads();
    // thread t: column t % hd over keys j = t / hd, t / hd + G, ... (G = 256 / hd groups)
    const int G = 256 / hd, d = tid % hd, g = tid / hd;
    float acc = 0.0f;
    if (g < G)
        for (int j = g; j < L; j += G) acc += sc[j] * ld(vb + static_cast<int64_t>(j) * ldkv, d);
    red[tid] = acc;
    __syncthreads();
    if (tid < hd) {
        float t = 0.0f;
        for (int u = 0; u < G; ++u) t += red[u * hd + tid];
        st(o + (static_cast<int64_t>(b) * S_new + i) * ldo + static_cast<int64_t>(h) * hd, tid, t * inv);
    }
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool mfma_ok(const void* q, const void* k, const void* v, int64_t ldq, const void* o, int64_t ldo, int64_t hd) {
    return (hd == 64 || hd == 128) && ldq % 8 == 0 && ldo % 8 == 0 && a16(q) && a16(k) && a16(v) && a16(o) &&
           ldq < (int64_t{1} << 24) && ldo < (int64_t{1} << 24);  // 32-bit copy offsets (Rows64)
}

template <typename T>
void fwd_simt(const void* q, const void* k, const void* v, int64_t ldq, int64_t ldk, void* o, int64_t ldo, float* lse,
              int64_t B, int64_t H, int64_t S, int64_t Sk, int64_t hd, bool causal, float scale, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((S + kSimtTile - 1) / kSimtTile), static_cast<unsigned>(H),
                    static_cast<unsigned>(B));
#define AIC_FWD_SIMT(HD_)                                                                                     \
    hipLaunchKernelGGL((attn_fwd_simt<T, HD_>), grid, dim3(64), 0, s, static_cast<const T*>(q),                \
                       static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk, static_cast<T*>(o), ldo, lse, \
                       static_cast<int>(H), static_cast<int>(S), static_cast<int>(Sk), scale, causal ? 1 : 0)
    if (hd == 16) AIC_FWD_SIMT(16);
    else if (hd == 32) AIC_FWD_SIMT(32);
    else if (hd == 64) AIC_FWD_SIMT(64);
    else if (hd == 128) AIC_FWD_SIMT(128);
    else AIC_THROW(NotImplemented, "attention: head_dim ", hd, " is not supported on this path");
#undef AIC_FWD_SIMT
    AIC_LAUNCH_CHECK("attn_fwd_simt");
}

template <typename T>
void bwd_simt(const void* q, const void* k, const void* v, int64_t ldq, int64_t ldk, const void* dout, int64_t ldo,
              const float* lse, const float* D, void* dq, int64_t ldd, void* dk, void* dv, int64_t lddk, int64_t B,
              int64_t H, int64_t S, int64_t Sk, int64_t hd, bool causal, float scale, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((S + kSimtTile - 1) / kSimtTile), static_cast<unsigned>(H),
                    static_cast<unsigned>(B));
    const dim3 gridk(static_cast<unsigned>((Sk + kSimtTile - 1) / kSimtTile), static_cast<unsigned>(H),
                     static_cast<unsigned>(B));
#define AIC_BWD_SIMT(HD_)                                                                                      \
    do {                                                                                                        \
        hipLaunchKernelGGL((attn_bwd_kv_simt<T, HD_>), gridk, dim3(64), 0, s, static_cast<const T*>(q),         \
                           static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk,                        \
                           static_cast<const T*>(dout), ldo, lse, D, static_cast<T*>(dk), static_cast<T*>(dv),   \
                           ldd, lddk, static_cast<int>(H), static_cast<int>(S), static_cast<int>(Sk), scale,    \
                           causal ? 1 : 0);                                                                      \
        if (S > 0)                                                                                              \
            hipLaunchKernelGGL((attn_bwd_q_simt<T, HD_>), grid, dim3(64), 0, s, static_cast<const T*>(q),       \
                               static_cast<const T*>(k), static_cast<const T*>(v), ldq, ldk,                    \
                               static_cast<const T*>(dout), ldo, lse, D, static_cast<T*>(dq), ldd,               \
                               static_cast<int>(H), static_cast<int>(S), static_cast<int>(Sk), scale,           \
                               causal ? 1 : 0);                                                                  \
    } while (0)
    if (hd == 16) AIC_BWD_SIMT(16);
    else if (hd == 32) AIC_BWD_SIMT(32);
    else if (hd == 64) AIC_BWD_SIMT(64);
    else if (hd == 128) AIC_BWD_SIMT(128);
    else AIC_THROW(NotImplemented, "attention: head_dim ", hd, " is not supported on this path");
#undef AIC_BWD_SIMT
    AIC_LAUNCH_CHECK("attn_bwd_simt");
}

}  // namespace

void attn_fwd(const void* q, const void* k, const void* v, int64_t ld_qkv, void* o, int64_t ld_o, float* lse,
              int64_t B, int64_t H, int64_t S, int64_t hd, bool causal, float scale, DType dt, hipStream_t s) {
    AIC_CHECK(B >= 0 && H > 0 && S >= 0 && hd > 0 && ld_qkv >= H * hd && ld_o >= H * hd, InvalidArgument,
              "attn_fwd: bad shape");
    AIC_CHECK(S < (1LL << 30) && B * S < (1LL << 31) && ((S + 127) / 128) * H * B < (1LL << 31), InvalidArgument,
              "attn_fwd: sequence too long");
    if (B == 0 || S == 0) return;
    if (dt == DType::BFloat16 && mfma_ok(q, k, v, ld_qkv, o, ld_o, hd)) {
        const dim3 grid(static_cast<unsigned>(((S + 127) / 128) * H * B));
        const float sl2 = scale * kLog2e;
        if (hd == 128)
            hipLaunchKernelGGL(attn_fwd_pipe<128>, grid, dim3(256), 0, s, static_cast<const bf16*>(q),
                               static_cast<const bf16*>(k), static_cast<const bf16*>(v), ld_qkv, static_cast<bf16*>(o),
                               ld_o, lse, static_cast<int>(H), static_cast<int>(S), sl2, causal ? 1 : 0);
        else
            hipLaunchKernelGGL(attn_fwd_pipe<64>, grid, dim3(256), 0, s, static_cast<const bf16*>(q),
                               static_cast<const bf16*>(k), static_cast<const bf16*>(v), ld_qkv, static_cast<bf16*>(o),
                               ld_o, lse, static_cast<int>(H), static_cast<int>(S), sl2, causal ? 1 : 0);
        AIC_LAUNCH_CHECK("attn_fwd_pipe");
        return;
    }
    if (dt == DType::Float32) fwd_simt<float>(q, k, v, ld_qkv, ld_qkv, o, ld_o, lse, B, H, S, S, hd, causal, scale, s);
    else if (dt == DType::BFloat16)
        fwd_simt<bf16>(q, k, v, ld_qkv, ld_qkv, o, ld_o, lse, B, H, S, S, hd, causal, scale, s);
    else AIC_THROW(DTypeMismatch, "attn_fwd: dtype must be f32 or bf16");
}

void attn_bwd(const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o, const void* dout,
              int64_t ld_o, const float* lse, void* dq, void* dk, void* dv, int64_t ld_d, int64_t B, int64_t H,
              int64_t S, int64_t hd, bool causal, float scale, DType dt, hipStream_t s, const float* rope_cos,
              const float* rope_sin) {
    AIC_CHECK((rope_cos == nullptr) == (rope_sin == nullptr), InvalidArgument, "attn_bwd: rope tables come in pairs");
    AIC_CHECK(B >= 0 && H > 0 && S >= 0 && hd > 0 && ld_qkv >= H * hd && ld_o >= H * hd && ld_d >= H * hd,
              InvalidArgument, "attn_bwd: bad shape");
    AIC_CHECK(S < (1LL << 30) && B * S < (1LL << 31) && ((S + 127) / 128) * H * B < (1LL << 31), InvalidArgument,
              "attn_bwd: sequence too long");
    if (B == 0 || S == 0) return;
    float* D = static_cast<float*>(stream_scratch(sizeof(float) * B * H * S, s));
    if (dt == DType::BFloat16 && mfma_ok(q, k, v, ld_qkv, dout, ld_o, hd) && ld_d % 8 == 0 && a16(dq) && a16(dk) &&
        a16(dv) && a16(o)) {
        // the dQ kernel computes D = rowsum(dO * O) for its queries and writes it for dK/dV
        const float sl2 = scale * kLog2e;
        const dim3 grid(static_cast<unsigned>(((S + 127) / 128) * H * B));
#define AIC_BWD_MFMA(HD_)                                                                                        \
    do {                                                                                                          \
        hipLaunchKernelGGL(attn_bwd_dq_mfma<HD_>, grid, dim3(256), 0, s, static_cast<const bf16*>(q),             \
                           static_cast<const bf16*>(k), static_cast<const bf16*>(v), ld_qkv,                       \
                           static_cast<const bf16*>(o), static_cast<const bf16*>(dout), ld_o, lse, D,              \
                           static_cast<bf16*>(dq), ld_d, static_cast<int>(H), static_cast<int>(S), sl2, scale,      \
                           causal ? 1 : 0, rope_cos, rope_sin);                                                    \
        AIC_LAUNCH_CHECK("attn_bwd_dq_mfma");                                                                      \
        hipLaunchKernelGGL(attn_bwd_dkdv_mfma<HD_>, grid, dim3(256), 0, s, static_cast<const bf16*>(q),           \
                           static_cast<const bf16*>(k), static_cast<const bf16*>(v), ld_qkv,                       \
                           static_cast<const bf16*>(dout), ld_o, lse, D, static_cast<bf16*>(dk),                   \
                           static_cast<bf16*>(dv), ld_d, static_cast<int>(H), static_cast<int>(S), sl2, scale,      \
                           causal ? 1 : 0, rope_cos, rope_sin);                                                    \
        AIC_LAUNCH_CHECK("attn_bwd_dkdv_mfma");                                                                    \
    } while (0)
        if (hd == 128) AIC_BWD_MFMA(128);
        else AIC_BWD_MFMA(64);
#undef AIC_BWD_MFMA
        return;
    }
    const int64_t waves = B * S * H;
    const unsigned dgrid = static_cast<unsigned>((waves * 64 + 255) / 256);
    const bool al16 = (reinterpret_cast<uintptr_t>(o) & 15u) == 0 && (reinterpret_cast<uintptr_t>(dout) & 15u) == 0;
    if (dt == DType::BFloat16 && ld_o % 8 == 0 && al16 && (hd == 32 || hd == 64 || hd == 128)) {
        const int64_t rpw = 64 / (hd / 8);  // rows per wave
        const unsigned g8 = static_cast<unsigned>(((waves + rpw - 1) / rpw * 64 + 255) / 256);
        const bf16* ob = static_cast<const bf16*>(o);
        const bf16* db = static_cast<const bf16*>(dout);
        if (hd == 128)
            hipLaunchKernelGGL(attn_dot_v8_k<128>, dim3(g8), dim3(256), 0, s, ob, db, ld_o, D, B * S,
                               static_cast<int>(H), static_cast<int>(S));
        else if (hd == 64)
            hipLaunchKernelGGL(attn_dot_v8_k<64>, dim3(g8), dim3(256), 0, s, ob, db, ld_o, D, B * S,
                               static_cast<int>(H), static_cast<int>(S));
        else
            hipLaunchKernelGGL(attn_dot_v8_k<32>, dim3(g8), dim3(256), 0, s, ob, db, ld_o, D, B * S,
                               static_cast<int>(H), static_cast<int>(S));
    } else if (dt == DType::BFloat16)
        hipLaunchKernelGGL(attn_dot_k<bf16>, dim3(dgrid), dim3(256), 0, s, static_cast<const bf16*>(o),
                           static_cast<const bf16*>(dout), ld_o, D, B * S, static_cast<int>(H), static_cast<int>(S),
                           static_cast<int>(hd));
    else if (dt == DType::Float32)
        hipLaunchKernelGGL(attn_dot_k<float>, dim3(dgrid), dim3(256), 0, s, static_cast<const float*>(o),
                           static_cast<const float*>(dout), ld_o, D, B * S, static_cast<int>(H), static_cast<int>(S),
                           static_cast<int>(hd));
    else
        AIC_THROW(DTypeMismatch, "attn_bwd: dtype must be f32 or bf16");
    AIC_LAUNCH_CHECK("attn_dot");

    if (dt == DType::Float32)
        bwd_simt<float>(q, k, v, ld_qkv, ld_qkv, dout, ld_o, lse, D, dq, ld_d, dk, dv, ld_d, B, H, S, S, hd, causal,
                        scale, s);
    else
        bwd_simt<bf16>(q, k, v, ld_qkv, ld_qkv, dout, ld_o, lse, D, dq, ld_d, dk, dv, ld_d, B, H, S, S, hd, causal,
                       scale, s);
    if (rope_cos) {  // the rotary embedding's adjoint as its own pass on these paths
        rope(dq, ld_d, B, S, H, hd, 0, rope_cos, rope_sin, true, dt, s);
        rope(dk, ld_d, B, S, H, hd, 0, rope_cos, rope_sin, true, dt, s);
    }
}

// Queries and keys of different lengths (launch_flash_attention_forward/backward_gpu take
// seq_len_q and seq_len_k, src/cuda/cuda_flash_attention.cuh:12-46): q, o, dO [B, Sq] token rows
// of H heads (leading dimensions ld_q, ld_o), k, v [B, Sk] rows (ld_k); causal as the reference's
// CPU path (src/ops/flash_attention.cpp:76-89, 170-260): query r sees keys c <= r.  The SIMT
// kernels (fp32 math) for any dtype; lse [B, H, Sq].
void attn_fwd_qk(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_k, void* o, int64_t ld_o,
                 float* lse, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t hd, bool causal, float scale,
                 DType dt, hipStream_t s) {
    AIC_CHECK(B >= 0 && H > 0 && Sq >= 0 && Sk >= 0 && hd > 0 && ld_q >= H * hd && ld_k >= H * hd && ld_o >= H * hd,
              InvalidArgument, "attn_fwd: bad shape");
    AIC_CHECK(Sq < (1LL << 30) && Sk < (1LL << 30) && B * std::max(Sq, Sk) < (1LL << 31), InvalidArgument,
              "attn_fwd: sequence too long");
    if (B == 0 || Sq == 0) return;
    AIC_CHECK(Sk > 0, InvalidArgument, "attn_fwd: no keys");
    if (dt == DType::Float32) fwd_simt<float>(q, k, v, ld_q, ld_k, o, ld_o, lse, B, H, Sq, Sk, hd, causal, scale, s);
    else if (dt == DType::BFloat16)
        fwd_simt<bf16>(q, k, v, ld_q, ld_k, o, ld_o, lse, B, H, Sq, Sk, hd, causal, scale, s);
    else AIC_THROW(DTypeMismatch, "attn_fwd: dtype must be f32 or bf16");
}

void attn_bwd_qk(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_k, const void* o,
                 const void* dout, int64_t ld_o, const float* lse, void* dq, int64_t ld_dq, void* dk, void* dv,
                 int64_t ld_dkv, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t hd, bool causal, float scale,
                 DType dt, hipStream_t s) {
    AIC_CHECK(B >= 0 && H > 0 && Sq >= 0 && Sk >= 0 && hd > 0 && ld_q >= H * hd && ld_k >= H * hd &&
                  ld_o >= H * hd && ld_dq >= H * hd && ld_dkv >= H * hd,
              InvalidArgument, "attn_bwd: bad shape");
    AIC_CHECK(Sq < (1LL << 30) && Sk < (1LL << 30) && B * std::max(Sq, Sk) < (1LL << 31), InvalidArgument,
              "attn_bwd: sequence too long");
    if (B == 0) return;
    AIC_CHECK(Sk > 0, InvalidArgument, "attn_bwd: no keys");
    AIC_CHECK(dt == DType::Float32 || dt == DType::BFloat16, DTypeMismatch, "attn_bwd: dtype must be f32 or bf16");
    // no queries: only the key kernel runs, and its empty query loop writes zero dK and dV
    float* D = static_cast<float*>(stream_scratch(sizeof(float) * std::max<int64_t>(B * H * Sq, 1), s));
    if (Sq > 0) {
        const unsigned dgrid = static_cast<unsigned>((B * Sq * H * 64 + 255) / 256);
        if (dt == DType::Float32)
            hipLaunchKernelGGL(attn_dot_k<float>, dim3(dgrid), dim3(256), 0, s, static_cast<const float*>(o),
                               static_cast<const float*>(dout), ld_o, D, B * Sq, static_cast<int>(H),
                               static_cast<int>(Sq), static_cast<int>(hd));
        else
            hipLaunchKernelGGL(attn_dot_k<bf16>, dim3(dgrid), dim3(256), 0, s, static_cast<const bf16*>(o),
                               static_cast<const bf16*>(dout), ld_o, D, B * Sq, static_cast<int>(H),
                               static_cast<int>(Sq), static_cast<int>(hd));
        AIC_LAUNCH_CHECK("attn_dot");
    }
    if (dt == DType::Float32)
        bwd_simt<float>(q, k, v, ld_q, ld_k, dout, ld_o, lse, D, dq, ld_dq, dk, dv, ld_dkv, B, H, Sq, Sk, hd, causal,
                        scale, s);
    else
        bwd_simt<bf16>(q, k, v, ld_q, ld_k, dout, ld_o, lse, D, dq, ld_dq, dk, dv, ld_dkv, B, H, Sq, Sk, hd, causal,
                       scale, s);
}

void attn_cached(const void* q, int64_t ldq, const void* kc, const void* vc, int64_t ldkv, int64_t cache_rows, void* o,
                 int64_t ldo, int64_t B, int64_t H, int64_t S_new, int64_t start_pos, int64_t hd, float scale, DType dt,
                 hipStream_t s) {
    AIC_CHECK(B >= 0 && H > 0 && S_new >= 0 && start_pos >= 0 && hd > 0 && hd <= 128 && 256 % hd == 0 &&
                  ldq >= H * hd && ldkv >= H * hd && ldo >= H * hd,
              InvalidArgument, "attn_cached: bad shape");
    AIC_CHECK(start_pos + S_new <= cache_rows && start_pos + S_new <= 16384, InvalidArgument,
              "attn_cached: the cache holds ", cache_rows, " positions (at most 16384), needed ", start_pos + S_new);
    if (B == 0 || S_new == 0) return;
    const dim3 grid(static_cast<unsigned>(S_new), static_cast<unsigned>(H), static_cast<unsigned>(B));
    const size_t lds = sizeof(float) * static_cast<size_t>(start_pos + S_new + 256);
    const int64_t bstride = cache_rows * ldkv;
    static bool configured = false;  // allow the scores of up to 16384 positions in LDS
    if (!configured) {
        AIC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_cached_k<bf16>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024));
        AIC_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_cached_k<float>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024));
        configured = true;
    }
    if (dt == DType::BFloat16)
        hipLaunchKernelGGL(attn_cached_k<bf16>, grid, dim3(256), lds, s, static_cast<const bf16*>(q), ldq,
                           static_cast<const bf16*>(kc), static_cast<const bf16*>(vc), ldkv, bstride,
                           static_cast<bf16*>(o), ldo, static_cast<int>(S_new), static_cast<int>(start_pos),
                           static_cast<int>(hd), scale);
    else if (dt == DType::Float32)
        hipLaunchKernelGGL(attn_cached_k<float>, grid, dim3(256), lds, s, static_cast<const float*>(q), ldq,
                           static_cast<const float*>(kc), static_cast<const float*>(vc), ldkv, bstride,
                           static_cast<float*>(o), ldo, static_cast<int>(S_new), static_cast<int>(start_pos),
                           static_cast<int>(hd), scale);
    else
        AIC_THROW(DTypeMismatch, "attn_cached: dtype must be f32 or bf16");
    AIC_LAUNCH_CHECK("attn_cached");
}

}  // namespace aic::hip
