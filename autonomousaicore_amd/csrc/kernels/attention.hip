// Causal flash attention forward/backward.
//
// Replaces launch_flash_attention_forward/backward_gpu (src/cuda/cuda_flash_attention.cu,
// one 64-thread block per query row, fp32, wrong for head_dim > 64) and the default
// materialised path of CausalSelfAttention (include/nn/attention.hpp:84-119).  Same
// mathematics: softmax(Q K^T * scale + causal mask) V with the row log-sum-exp saved.
//
// bf16 path (head_dim 64 / 128), v_mfma_f32_32x32x16_bf16, wave64:
//   forward   one block = 128 queries (4 waves x 32), K/V tiles of 64 keys double-buffered
//             in LDS.  Each wave computes S^T = K Q^T so that a lane owns one query: the row
//             max/sum need one cross-half exchange (lane ^ 32) and the rescale of the
//             output accumulator O^T is per lane.  P^T feeds O^T += V^T P^T straight from
//             the accumulator registers: the MFMA k-order is permuted identically on the A
//             side (V^T read from a transposed LDS tile with two 8-byte reads).
//   backward  two kernels, no atomics (deterministic):
//             dK/dV: one block = 128 keys (4 waves x 32) looping over 64-query tiles; S and
//             dP are computed as [query x key] so a lane owns a key and P / dS feed
//             dV^T += dO^T P and dK^T += Q^T dS from registers.
//             dQ:   one block = 128 queries looping over 64-key tiles (dQ^T += K^T dS^T).
// fp32 path (the fp32 reference configuration, head_dim <= 64): SIMT kernels, fp32 math.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------------------
// LDS layouts
//   row-major "K-contiguous" tile [rows][HD]: 16-byte chunks XOR-swizzled per row
//   transposed tile [HD][64]: 8-byte chunks XOR-swizzled per row
// ---------------------------------------------------------------------------------------
template <int HD>
__device__ __forceinline__ int swz16(int row) {
    constexpr int NC = HD / 8;
    constexpr int SH = NC == 16 ? 4 : (NC == 8 ? 3 : 2);
    return (row ^ (row >> SH)) & (NC - 1);
}
__device__ __forceinline__ int swz8(int row) { return (row ^ (row >> 4)) & 15; }

template <int HD>
__device__ __forceinline__ bf16x8 read_row_frag(const bf16* t, int row, int chunk) {
    return *reinterpret_cast<const bf16x8*>(t + row * HD + ((chunk ^ swz16<HD>(row)) << 3));
}
// A-operand fragment from a transposed [HD][64] tile for the permuted 16-wide k-step ks:
// elements 0..3 = columns 16ks + 4h + (0..3), elements 4..7 = columns 16ks + 8 + 4h + (0..3).
__device__ __forceinline__ bf16x8 read_t_frag(const bf16* t, int row, int ks, int h) {
    const int ca = 4 * ks + h, cb = 4 * ks + 2 + h;
    const int sw = swz8(row);
    const uint2 a = *reinterpret_cast<const uint2*>(t + row * 64 + ((ca ^ sw) << 2));
    const uint2 b = *reinterpret_cast<const uint2*>(t + row * 64 + ((cb ^ sw) << 2));
    uint4 r = make_uint4(a.x, a.y, b.x, b.y);
    return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// 8 rows x 8 columns (16 bytes per row) held as r[0..7] -> write column block into a
// transposed [HD][64] tile: output row (col0 + j) gets the 8 values r[0..7][j] at tile
// columns row0 .. row0+7.
__device__ __forceinline__ void store_transposed8(bf16* t, const uint4* r, int col0, int row0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t w0 = __builtin_amdgcn_perm(word(r[1], j >> 1), word(r[0], j >> 1), sel);
        const uint32_t w1 = __builtin_amdgcn_perm(word(r[3], j >> 1), word(r[2], j >> 1), sel);
        const uint32_t w2 = __builtin_amdgcn_perm(word(r[5], j >> 1), word(r[4], j >> 1), sel);
        const uint32_t w3 = __builtin_amdgcn_perm(word(r[7], j >> 1), word(r[6], j >> 1), sel);
        const int row = col0 + j;
        const int sw = swz8(row);
        const int c = row0 >> 2;  // 8-byte chunk index of the first 4 columns
        *reinterpret_cast<uint2*>(t + row * 64 + ((c ^ sw) << 2)) = make_uint2(w0, w1);
        *reinterpret_cast<uint2*>(t + row * 64 + (((c + 1) ^ sw) << 2)) = make_uint2(w2, w3);
    }
}

__device__ __forceinline__ bf16x8 pack_bf16x8(const f32x16& a, int off) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = f2bf(a[off + i]);
    return r;
}

__device__ __forceinline__ uint4 ldg16(const bf16* p, bool ok) {
    return ok ? *reinterpret_cast<const uint4*>(p) : make_uint4(0, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256, 1) void attn_fwd_mfma(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                        const bf16* __restrict__ v, int64_t ldq, bf16* __restrict__ o,
                                                        int64_t ldo, float* __restrict__ lse, int H, int S,
                                                        float scale_log2, int causal) {
    constexpr int BQ = 128, BKV = 64, NC = HD / 8, KS = HD / 16, OB = HD / 32;
    __shared__ __attribute__((aligned(16))) bf16 sK[2][BKV * HD];
    __shared__ __attribute__((aligned(16))) bf16 sVt[2][HD * BKV];

    const int nq = (S + BQ - 1) / BQ;
    const int qb = nq - 1 - static_cast<int>(blockIdx.x);
    const int h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
    const int q0 = qb * BQ;
    const int qw = q0 + wave * 32;
    const int myq = qw + (lane & 31);
    const int64_t tok0 = static_cast<int64_t>(b) * S;
    const bf16* kb = k + tok0 * ldq + static_cast<int64_t>(h) * HD;
    const bf16* vb = v + tok0 * ldq + static_cast<int64_t>(h) * HD;

    bf16x8 qf[KS];
    {
        const bf16* qp = q + (tok0 + myq) * ldq + static_cast<int64_t>(h) * HD + 8 * hl;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) qf[kk] = __builtin_bit_cast(bf16x8, ldg16(qp + 16 * kk, myq < S));
    }

    f32x16 oacc[OB];
#pragma unroll
    for (int i = 0; i < OB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[i][e] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    const int kv_end = causal ? min(S, q0 + BQ) : S;
    const int ntiles = (kv_end + BKV - 1) / BKV;

    // loaders: K rows (NC/4 chunks per thread); V 8x8 blocks (threads < 8*NC)
    constexpr int KCH = BKV * NC / 256;
    uint4 rk[KCH], rv[8];
    auto gload = [&](int t) {
        const int k0 = t * BKV;
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int c = threadIdx.x + 256 * i;
            const int row = c / NC, ch = c % NC;
            rk[i] = ldg16(kb + static_cast<int64_t>(k0 + row) * ldq + ch * 8, k0 + row < S);
        }
        if (threadIdx.x < 8 * NC) {
            const int kg = threadIdx.x & 7, hc = threadIdx.x >> 3;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int key = k0 + kg * 8 + i;
                rv[i] = ldg16(vb + static_cast<int64_t>(key) * ldq + hc * 8, key < S);
            }
        }
    };
    auto sstore = [&](int st) {
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int c = threadIdx.x + 256 * i;
            const int row = c / NC, ch = c % NC;
            *reinterpret_cast<uint4*>(&sK[st][row * HD + ((ch ^ swz16<HD>(row)) << 3)]) = rk[i];
        }
        if (threadIdx.x < 8 * NC) {
            const int kg = threadIdx.x & 7, hc = threadIdx.x >> 3;
            store_transposed8(sVt[st], rv, hc * 8, kg * 8);
        }
    };

    if (ntiles > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int st = t & 1;
        if (t + 1 < ntiles) gload(t + 1);
        const int k0 = t * BKV;
        const bool active = !causal || (k0 <= qw + 31);
        if (active) {
            f32x16 s[2];
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                for (int e = 0; e < 16; ++e) s[jb][e] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
                for (int jb = 0; jb < 2; ++jb) {
                    const bf16x8 kf = read_row_frag<HD>(sK[st], jb * 32 + (lane & 31), 2 * kk + hl);
                    s[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[jb], 0, 0, 0);
                }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = k0 + jb * 32 + 8 * (e >> 2) + 4 * hl + (e & 3);
                    float x = s[jb][e] * scale_log2;
                    if ((causal && key > myq) || key >= S) x = -INFINITY;
                    s[jb][e] = x;
                    mx = fmaxf(mx, x);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_run, mx);
            const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            float rs = 0.0f;
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float p = (s[jb][e] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s[jb][e] - m_new);
                    s[jb][e] = p;
                    rs += p;
                }
            rs += __shfl_xor(rs, 32, 64);
            l_run = l_run * alpha + rs;
            m_run = m_new;
#pragma unroll
            for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[ob][e] *= alpha;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 pf = pack_bf16x8(s[ks >> 1], 8 * (ks & 1));
#pragma unroll
                for (int ob = 0; ob < OB; ++ob) {
                    const bf16x8 vf = read_t_frag(sVt[st], ob * 32 + (lane & 31), ks, hl);
                    oacc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, oacc[ob], 0, 0, 0);
                }
            }
        }
        if (t + 1 < ntiles) sstore(st ^ 1);
        __syncthreads();
    }

    if (myq < S) {
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
        bf16* op = o + (tok0 + myq) * ldo + static_cast<int64_t>(h) * HD;
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = ob * 32 + 8 * g + 4 * hl;
                const uint32_t w0 = static_cast<uint32_t>(f2bf_bits(oacc[ob][4 * g] * inv)) |
                                    (static_cast<uint32_t>(f2bf_bits(oacc[ob][4 * g + 1] * inv)) << 16);
                const uint32_t w1 = static_cast<uint32_t>(f2bf_bits(oacc[ob][4 * g + 2] * inv)) |
                                    (static_cast<uint32_t>(f2bf_bits(oacc[ob][4 * g + 3] * inv)) << 16);
                *reinterpret_cast<uint2*>(op + d0) = make_uint2(w0, w1);
            }
        if (hl == 0) lse[(static_cast<int64_t>(b) * H + h) * S + myq] = (m_run + log2f(l_run)) * kLn2;
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

// ---------------------------------------------------------------------------------------
// Backward: dK, dV
// ---------------------------------------------------------------------------------------
template <int HD>
struct BwdKVSmem {
    bf16 q[64 * HD];
    bf16 qt[HD * 64];
    bf16 dO[64 * HD];
    bf16 dOt[HD * 64];
    float lse2[64];
    float D[64];
};

template <int HD>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_mfma(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int64_t ldq,
    const bf16* __restrict__ dout, int64_t ldo, const float* __restrict__ lse, const float* __restrict__ Dg,
    bf16* __restrict__ dk, bf16* __restrict__ dv, int64_t ldd, int H, int S, float scale_log2, float scale,
    int causal) {
    constexpr int BQ = 64, BKV = 128, NC = HD / 8, KS = HD / 16, OB = HD / 32;
    __shared__ __attribute__((aligned(16))) BwdKVSmem<HD> sm[2];

    const int nkv = (S + BKV - 1) / BKV;
    const int kb_ = nkv - 1 - static_cast<int>(blockIdx.x);  // kv tiles with most work first (lowest keys)
    const int kblk = causal ? (nkv - 1 - kb_) : kb_;
    const int h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
    const int k0 = kblk * BKV;
    const int kw = k0 + wave * 32;
    const int mykey = kw + (lane & 31);
    const int64_t tok0 = static_cast<int64_t>(b) * S;
    const int64_t hoff = static_cast<int64_t>(h) * HD;

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
    f32x16 dvt[OB], dkt[OB];
#pragma unroll
    for (int i = 0; i < OB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            dvt[i][e] = 0.0f;
            dkt[i][e] = 0.0f;
        }

    const int nq = (S + BQ - 1) / BQ;
    const int qt_begin = causal ? (k0 / BQ) : 0;
    const float* lse_bh = lse + (static_cast<int64_t>(b) * H + h) * S;
    const float* D_bh = Dg + (static_cast<int64_t>(b) * H + h) * S;

    // loader: threads [0, 8NC) load Q 8x8 blocks, threads [128, 128 + 8NC) load dO blocks.
    uint4 r[8];
    float rl = 0.0f, rd = 0.0f;
    const int half = threadIdx.x >> 7, tl = threadIdx.x & 127;
    auto gload = [&](int qt) {
        const int qs = qt * BQ;
        if (tl < 8 * NC) {
            const int rg = tl & 7, hc = tl >> 3;
            const bf16* src = half == 0 ? q : dout;
            const int64_t lds = half == 0 ? ldq : ldo;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = qs + rg * 8 + i;
                r[i] = ldg16(src + (tok0 + row) * lds + hoff + hc * 8, row < S);
            }
        }
        if (threadIdx.x < 64) {
            const int row = qs + threadIdx.x;
            rl = row < S ? lse_bh[row] * kLog2e : 0.0f;
            rd = row < S ? D_bh[row] : 0.0f;
        }
    };
    auto sstore = [&](int st) {
        if (tl < 8 * NC) {
            const int rg = tl & 7, hc = tl >> 3;
            bf16* rowt = half == 0 ? sm[st].q : sm[st].dO;
            bf16* trt = half == 0 ? sm[st].qt : sm[st].dOt;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = rg * 8 + i;
                *reinterpret_cast<uint4*>(rowt + row * HD + ((hc ^ swz16<HD>(row)) << 3)) = r[i];
            }
            store_transposed8(trt, r, hc * 8, rg * 8);
        }
        if (threadIdx.x < 64) {
            sm[st].lse2[threadIdx.x] = rl;
            sm[st].D[threadIdx.x] = rd;
        }
    };

    if (qt_begin < nq) {
        gload(qt_begin);
        sstore(0);
    }
    __syncthreads();

    for (int qt = qt_begin; qt < nq; ++qt) {
        const int st = (qt - qt_begin) & 1;
        if (qt + 1 < nq) gload(qt + 1);
        const int qs = qt * BQ;
        const bool active = !causal || (qs + BQ - 1 >= kw);
        if (active) {
            f32x16 s[2], dp[2];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    s[mb][e] = 0.0f;
                    dp[mb][e] = 0.0f;
                }
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    const bf16x8 qa = read_row_frag<HD>(sm[st].q, mb * 32 + (lane & 31), 2 * kk + hl);
                    s[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, kf[kk], s[mb], 0, 0, 0);
                    const bf16x8 da = read_row_frag<HD>(sm[st].dO, mb * 32 + (lane & 31), 2 * kk + hl);
                    dp[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da, vf[kk], dp[mb], 0, 0, 0);
                }
            // s[mb][e]: query qs + 32mb + 8(e/4) + 4hl + e%4, key mykey
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int qi = mb * 32 + 8 * (e >> 2) + 4 * hl + (e & 3);
                    const int qq = qs + qi;
                    const bool valid = (qq < S) && (mykey < S) && (!causal || mykey <= qq);
                    const float p = valid ? __builtin_amdgcn_exp2f(s[mb][e] * scale_log2 - sm[st].lse2[qi]) : 0.0f;
                    s[mb][e] = p;
                    dp[mb][e] = p * (dp[mb][e] - sm[st].D[qi]);
                }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 pf = pack_bf16x8(s[ks >> 1], 8 * (ks & 1));
                const bf16x8 dsf = pack_bf16x8(dp[ks >> 1], 8 * (ks & 1));
#pragma unroll
                for (int ob = 0; ob < OB; ++ob) {
                    const int hrow = ob * 32 + (lane & 31);
                    const bf16x8 doa = read_t_frag(sm[st].dOt, hrow, ks, hl);
                    dvt[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(doa, pf, dvt[ob], 0, 0, 0);
                    const bf16x8 qa = read_t_frag(sm[st].qt, hrow, ks, hl);
                    dkt[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, dsf, dkt[ob], 0, 0, 0);
                }
            }
        }
        if (qt + 1 < nq) sstore(st ^ 1);
        __syncthreads();
    }

    if (mykey < S) {
        bf16* dkp = dk + (tok0 + mykey) * ldd + hoff;
        bf16* dvp = dv + (tok0 + mykey) * ldd + hoff;
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = ob * 32 + 8 * g + 4 * hl;
                uint32_t wk[2], wv[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    wk[u] = static_cast<uint32_t>(f2bf_bits(dkt[ob][4 * g + 2 * u] * scale)) |
                            (static_cast<uint32_t>(f2bf_bits(dkt[ob][4 * g + 2 * u + 1] * scale)) << 16);
                    wv[u] = static_cast<uint32_t>(f2bf_bits(dvt[ob][4 * g + 2 * u])) |
                            (static_cast<uint32_t>(f2bf_bits(dvt[ob][4 * g + 2 * u + 1])) << 16);
                }
                *reinterpret_cast<uint2*>(dkp + d0) = make_uint2(wk[0], wk[1]);
                *reinterpret_cast<uint2*>(dvp + d0) = make_uint2(wv[0], wv[1]);
            }
    }
}

// ---------------------------------------------------------------------------------------
// Backward: dQ
// ---------------------------------------------------------------------------------------
template <int HD>
struct BwdQSmem {
    bf16 k[64 * HD];
    bf16 kt[HD * 64];
    bf16 v[64 * HD];
};

template <int HD>
__global__ __launch_bounds__(256, 1) void attn_bwd_dq_mfma(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                           const bf16* __restrict__ v, int64_t ldq,
                                                           const bf16* __restrict__ dout, int64_t ldo,
                                                           const float* __restrict__ lse, const float* __restrict__ Dg,
                                                           bf16* __restrict__ dq, int64_t ldd, int H, int S,
                                                           float scale_log2, float scale, int causal) {
    constexpr int BQ = 128, BKV = 64, NC = HD / 8, KS = HD / 16, OB = HD / 32;
    __shared__ __attribute__((aligned(16))) BwdQSmem<HD> sm[2];

    const int nq = (S + BQ - 1) / BQ;
    const int qb = nq - 1 - static_cast<int>(blockIdx.x);
    const int h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
    const int q0 = qb * BQ;
    const int qw = q0 + wave * 32;
    const int myq = qw + (lane & 31);
    const int64_t tok0 = static_cast<int64_t>(b) * S;
    const int64_t hoff = static_cast<int64_t>(h) * HD;

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
    const float my_lse2 = myq < S ? lse[(static_cast<int64_t>(b) * H + h) * S + myq] * kLog2e : 0.0f;
    const float my_D = myq < S ? Dg[(static_cast<int64_t>(b) * H + h) * S + myq] : 0.0f;

    f32x16 dqt[OB];
#pragma unroll
    for (int i = 0; i < OB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) dqt[i][e] = 0.0f;

    const int kv_end = causal ? min(S, q0 + BQ) : S;
    const int ntiles = (kv_end + BKV - 1) / BKV;

    // loader: threads [0, 8NC) load K as 8x8 blocks (both layouts); threads [128, 256) load V rows
    uint4 r[8];
    const int half = threadIdx.x >> 7, tl = threadIdx.x & 127;
    constexpr int VCH = BKV * NC / 128;
    auto gload = [&](int t) {
        const int k0 = t * BKV;
        if (half == 0) {
            if (tl < 8 * NC) {
                const int rg = tl & 7, hc = tl >> 3;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int row = k0 + rg * 8 + i;
                    r[i] = ldg16(k + (tok0 + row) * ldq + hoff + hc * 8, row < S);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < VCH; ++i) {
                const int c = tl + 128 * i;
                const int row = c / NC, ch = c % NC;
                r[i] = ldg16(v + (tok0 + k0 + row) * ldq + hoff + ch * 8, k0 + row < S);
            }
        }
    };
    auto sstore = [&](int st) {
        if (half == 0) {
            if (tl < 8 * NC) {
                const int rg = tl & 7, hc = tl >> 3;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int row = rg * 8 + i;
                    *reinterpret_cast<uint4*>(sm[st].k + row * HD + ((hc ^ swz16<HD>(row)) << 3)) = r[i];
                }
                store_transposed8(sm[st].kt, r, hc * 8, rg * 8);
            }
        } else {
#pragma unroll
            for (int i = 0; i < VCH; ++i) {
                const int c = tl + 128 * i;
                const int row = c / NC, ch = c % NC;
                *reinterpret_cast<uint4*>(sm[st].v + row * HD + ((ch ^ swz16<HD>(row)) << 3)) = r[i];
            }
        }
    };

    if (ntiles > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int st = t & 1;
        if (t + 1 < ntiles) gload(t + 1);
        const int k0 = t * BKV;
        const bool active = !causal || (k0 <= qw + 31);
        if (active) {
            f32x16 s[2], dp[2];
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    s[jb][e] = 0.0f;
                    dp[jb][e] = 0.0f;
                }
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
#pragma unroll
                for (int jb = 0; jb < 2; ++jb) {
                    const bf16x8 ka = read_row_frag<HD>(sm[st].k, jb * 32 + (lane & 31), 2 * kk + hl);
                    s[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[kk], s[jb], 0, 0, 0);
                    const bf16x8 va = read_row_frag<HD>(sm[st].v, jb * 32 + (lane & 31), 2 * kk + hl);
                    dp[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, df[kk], dp[jb], 0, 0, 0);
                }
#pragma unroll
            for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = k0 + jb * 32 + 8 * (e >> 2) + 4 * hl + (e & 3);
                    const bool valid = (key < S) && (myq < S) && (!causal || key <= myq);
                    const float p = valid ? __builtin_amdgcn_exp2f(s[jb][e] * scale_log2 - my_lse2) : 0.0f;
                    dp[jb][e] = p * (dp[jb][e] - my_D);
                }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 dsf = pack_bf16x8(dp[ks >> 1], 8 * (ks & 1));
#pragma unroll
                for (int ob = 0; ob < OB; ++ob) {
                    const bf16x8 ka = read_t_frag(sm[st].kt, ob * 32 + (lane & 31), ks, hl);
                    dqt[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, dsf, dqt[ob], 0, 0, 0);
                }
            }
        }
        if (t + 1 < ntiles) sstore(st ^ 1);
        __syncthreads();
    }

    if (myq < S) {
        bf16* dqp = dq + (tok0 + myq) * ldd + hoff;
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = ob * 32 + 8 * g + 4 * hl;
                const uint32_t w0 = static_cast<uint32_t>(f2bf_bits(dqt[ob][4 * g] * scale)) |
                                    (static_cast<uint32_t>(f2bf_bits(dqt[ob][4 * g + 1] * scale)) << 16);
                const uint32_t w1 = static_cast<uint32_t>(f2bf_bits(dqt[ob][4 * g + 2] * scale)) |
                                    (static_cast<uint32_t>(f2bf_bits(dqt[ob][4 * g + 3] * scale)) << 16);
                *reinterpret_cast<uint2*>(dqp + d0) = make_uint2(w0, w1);
            }
    }
}

// ---------------------------------------------------------------------------------------
// SIMT path (fp32 configuration, any dtype, head_dim <= 64): one thread per query row
// (forward, dQ) or key row (dK, dV); fp32 math; K/V or Q/dO tiles staged in LDS.
// ---------------------------------------------------------------------------------------
constexpr int kSimtTile = 64;

template <typename T, int HD>
__global__ __launch_bounds__(64) void attn_fwd_simt(const T* __restrict__ q, const T* __restrict__ k,
                                                    const T* __restrict__ v, int64_t ldq, T* __restrict__ o,
                                                    int64_t ldo, float* __restrict__ lse, int H, int S, float scale,
                                                    int causal) {
    __shared__ float sk[kSimtTile][HD + 1];
    __shared__ float sv[kSimtTile][HD + 1];
    const int h = blockIdx.y, b = blockIdx.z;
    const int qi = blockIdx.x * kSimtTile + threadIdx.x;
    const int64_t tok0 = static_cast<int64_t>(b) * S;
    const int64_t hoff = static_cast<int64_t>(h) * HD;
    float qv[HD], acc[HD];
    for (int d = 0; d < HD; ++d) {
        qv[d] = qi < S ? ld(q, (tok0 + qi) * ldq + hoff + d) : 0.0f;
        acc[d] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    const int kend = causal ? min(S, static_cast<int>((blockIdx.x + 1) * kSimtTile)) : S;
    for (int k0 = 0; k0 < kend; k0 += kSimtTile) {
        __syncthreads();
        for (int e = threadIdx.x; e < kSimtTile * HD; e += 64) {
            const int r = e / HD, d = e % HD;
            const int key = k0 + r;
            sk[r][d] = key < S ? ld(k, (tok0 + key) * ldq + hoff + d) : 0.0f;
            sv[r][d] = key < S ? ld(v, (tok0 + key) * ldq + hoff + d) : 0.0f;
        }
        __syncthreads();
        if (qi >= S) continue;
        for (int r = 0; r < kSimtTile; ++r) {
            const int key = k0 + r;
            if (key >= S || (causal && key > qi)) break;
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
                                                       const T* __restrict__ v, int64_t ldq, const T* __restrict__ dout,
                                                       int64_t ldo, const float* __restrict__ lse,
                                                       const float* __restrict__ Dg, T* dk, T* dv, int64_t ldd, int H,
                                                       int S, float scale, int causal) {
    __shared__ float sq[kSimtTile][HD + 1];
    __shared__ float sdo[kSimtTile][HD + 1];
    __shared__ float sl[kSimtTile], sD[kSimtTile];
    const int h = blockIdx.y, b = blockIdx.z;
    const int kj = blockIdx.x * kSimtTile + threadIdx.x;
    const int64_t tok0 = static_cast<int64_t>(b) * S;
    const int64_t hoff = static_cast<int64_t>(h) * HD;
    const float* lse_bh = lse + (static_cast<int64_t>(b) * H + h) * S;
    const float* D_bh = Dg + (static_cast<int64_t>(b) * H + h) * S;
    float kv_[HD], vv[HD], dka[HD], dva[HD];
    for (int d = 0; d < HD; ++d) {
        kv_[d] = kj < S ? ld(k, (tok0 + kj) * ldq + hoff + d) : 0.0f;
        vv[d] = kj < S ? ld(v, (tok0 + kj) * ldq + hoff + d) : 0.0f;
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
        if (kj >= S) continue;
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
    if (kj < S)
        for (int d = 0; d < HD; ++d) {
            st(dk, (tok0 + kj) * ldd + hoff + d, dka[d] * scale);
            st(dv, (tok0 + kj) * ldd + hoff + d, dva[d]);
        }
}

template <typename T, int HD>
__global__ __launch_bounds__(64) void attn_bwd_q_simt(const T* __restrict__ q, const T* __restrict__ k,
                                                      const T* __restrict__ v, int64_t ldq, const T* __restrict__ dout,
                                                      int64_t ldo, const float* __restrict__ lse,
                                                      const float* __restrict__ Dg, T* dq, int64_t ldd, int H, int S,
                                                      float scale, int causal) {
    __shared__ float sk[kSimtTile][HD + 1];
    __shared__ float sv[kSimtTile][HD + 1];
    const int h = blockIdx.y, b = blockIdx.z;
    const int qi = blockIdx.x * kSimtTile + threadIdx.x;
    const int64_t tok0 = static_cast<int64_t>(b) * S;
    const int64_t hoff = static_cast<int64_t>(h) * HD;
    float qv[HD], dov[HD], acc[HD];
    for (int d = 0; d < HD; ++d) {
        qv[d] = qi < S ? ld(q, (tok0 + qi) * ldq + hoff + d) : 0.0f;
        dov[d] = qi < S ? ld(dout, (tok0 + qi) * ldo + hoff + d) : 0.0f;
        acc[d] = 0.0f;
    }
    const float l = qi < S ? lse[(static_cast<int64_t>(b) * H + h) * S + qi] : 0.0f;
    const float Dq = qi < S ? Dg[(static_cast<int64_t>(b) * H + h) * S + qi] : 0.0f;
    const int kend = causal ? min(S, static_cast<int>((blockIdx.x + 1) * kSimtTile)) : S;
    for (int k0 = 0; k0 < kend; k0 += kSimtTile) {
        __syncthreads();
        for (int e = threadIdx.x; e < kSimtTile * HD; e += 64) {
            const int r = e / HD, d = e % HD;
            const int key = k0 + r;
            sk[r][d] = key < S ? ld(k, (tok0 + key) * ldq + hoff + d) : 0.0f;
            sv[r][d] = key < S ? ld(v, (tok0 + key) * ldq + hoff + d) : 0.0f;
        }
        __syncthreads();
        if (qi >= S) continue;
        for (int r = 0; r < kSimtTile; ++r) {
            const int key = k0 + r;
            if (key >= S || (causal && key > qi)) break;
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

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool mfma_ok(const void* q, const void* k, const void* v, int64_t ldq, const void* o, int64_t ldo, int64_t hd) {
    return (hd == 64 || hd == 128) && ldq % 8 == 0 && ldo % 8 == 0 && a16(q) && a16(k) && a16(v) && a16(o);
}

template <typename T>
void fwd_simt(const void* q, const void* k, const void* v, int64_t ldq, void* o, int64_t ldo, float* lse, int64_t B,
              int64_t H, int64_t S, int64_t hd, bool causal, float scale, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((S + kSimtTile - 1) / kSimtTile), static_cast<unsigned>(H),
                    static_cast<unsigned>(B));
#define AIC_FWD_SIMT(HD_)                                                                                     \
    hipLaunchKernelGGL((attn_fwd_simt<T, HD_>), grid, dim3(64), 0, s, static_cast<const T*>(q),                \
                       static_cast<const T*>(k), static_cast<const T*>(v), ldq, static_cast<T*>(o), ldo, lse,     \
                       static_cast<int>(H), static_cast<int>(S), scale, causal ? 1 : 0)
    if (hd == 16) AIC_FWD_SIMT(16);
    else if (hd == 32) AIC_FWD_SIMT(32);
    else if (hd == 64) AIC_FWD_SIMT(64);
    else AIC_THROW(NotImplemented, "attention: head_dim ", hd, " is not supported on this path");
#undef AIC_FWD_SIMT
    AIC_LAUNCH_CHECK("attn_fwd_simt");
}

template <typename T>
void bwd_simt(const void* q, const void* k, const void* v, int64_t ldq, const void* dout, int64_t ldo, const float* lse,
              const float* D, void* dq, void* dk, void* dv, int64_t ldd, int64_t B, int64_t H, int64_t S, int64_t hd,
              bool causal, float scale, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((S + kSimtTile - 1) / kSimtTile), static_cast<unsigned>(H),
                    static_cast<unsigned>(B));
#define AIC_BWD_SIMT(HD_)                                                                                      \
    do {                                                                                                        \
        hipLaunchKernelGGL((attn_bwd_kv_simt<T, HD_>), grid, dim3(64), 0, s, static_cast<const T*>(q),          \
                           static_cast<const T*>(k), static_cast<const T*>(v), ldq, static_cast<const T*>(dout), \
                           ldo, lse, D, static_cast<T*>(dk), static_cast<T*>(dv), ldd, static_cast<int>(H),      \
                           static_cast<int>(S), scale, causal ? 1 : 0);                                          \
        hipLaunchKernelGGL((attn_bwd_q_simt<T, HD_>), grid, dim3(64), 0, s, static_cast<const T*>(q),           \
                           static_cast<const T*>(k), static_cast<const T*>(v), ldq, static_cast<const T*>(dout), \
                           ldo, lse, D, static_cast<T*>(dq), ldd, static_cast<int>(H), static_cast<int>(S),      \
                           scale, causal ? 1 : 0);                                                               \
    } while (0)
    if (hd == 16) AIC_BWD_SIMT(16);
    else if (hd == 32) AIC_BWD_SIMT(32);
    else if (hd == 64) AIC_BWD_SIMT(64);
    else AIC_THROW(NotImplemented, "attention: head_dim ", hd, " is not supported on this path");
#undef AIC_BWD_SIMT
    AIC_LAUNCH_CHECK("attn_bwd_simt");
}

}  // namespace

void attn_fwd(const void* q, const void* k, const void* v, int64_t ld_qkv, void* o, int64_t ld_o, float* lse,
              int64_t B, int64_t H, int64_t S, int64_t hd, bool causal, float scale, DType dt, hipStream_t s) {
    AIC_CHECK(B >= 0 && H > 0 && S >= 0 && hd > 0 && ld_qkv >= H * hd && ld_o >= H * hd, InvalidArgument,
              "attn_fwd: bad shape");
    AIC_CHECK(S < (1LL << 30) && B * S < (1LL << 31), InvalidArgument, "attn_fwd: sequence too long");
    if (B == 0 || S == 0) return;
    if (dt == DType::BFloat16 && mfma_ok(q, k, v, ld_qkv, o, ld_o, hd)) {
        const dim3 grid(static_cast<unsigned>((S + 127) / 128), static_cast<unsigned>(H), static_cast<unsigned>(B));
        const float sl2 = scale * kLog2e;
        if (hd == 128)
            hipLaunchKernelGGL(attn_fwd_mfma<128>, grid, dim3(256), 0, s, static_cast<const bf16*>(q),
                               static_cast<const bf16*>(k), static_cast<const bf16*>(v), ld_qkv, static_cast<bf16*>(o),
                               ld_o, lse, static_cast<int>(H), static_cast<int>(S), sl2, causal ? 1 : 0);
        else
            hipLaunchKernelGGL(attn_fwd_mfma<64>, grid, dim3(256), 0, s, static_cast<const bf16*>(q),
                               static_cast<const bf16*>(k), static_cast<const bf16*>(v), ld_qkv, static_cast<bf16*>(o),
                               ld_o, lse, static_cast<int>(H), static_cast<int>(S), sl2, causal ? 1 : 0);
        AIC_LAUNCH_CHECK("attn_fwd_mfma");
        return;
    }
    if (dt == DType::Float32) fwd_simt<float>(q, k, v, ld_qkv, o, ld_o, lse, B, H, S, hd, causal, scale, s);
    else if (dt == DType::BFloat16) fwd_simt<bf16>(q, k, v, ld_qkv, o, ld_o, lse, B, H, S, hd, causal, scale, s);
    else AIC_THROW(DTypeMismatch, "attn_fwd: dtype must be f32 or bf16");
}

void attn_bwd(const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o, const void* dout,
              int64_t ld_o, const float* lse, void* dq, void* dk, void* dv, int64_t ld_d, int64_t B, int64_t H,
              int64_t S, int64_t hd, bool causal, float scale, DType dt, hipStream_t s) {
    AIC_CHECK(B >= 0 && H > 0 && S >= 0 && hd > 0 && ld_qkv >= H * hd && ld_o >= H * hd && ld_d >= H * hd,
              InvalidArgument, "attn_bwd: bad shape");
    AIC_CHECK(S < (1LL << 30) && B * S < (1LL << 31), InvalidArgument, "attn_bwd: sequence too long");
    if (B == 0 || S == 0) return;
    DeviceBuffer Dbuf(sizeof(float) * B * H * S, s);
    float* D = Dbuf.as<float>();
    const int64_t waves = B * S * H;
    const unsigned dgrid = static_cast<unsigned>((waves * 64 + 255) / 256);
    if (dt == DType::BFloat16)
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

    if (dt == DType::BFloat16 && mfma_ok(q, k, v, ld_qkv, dout, ld_o, hd) && ld_d % 8 == 0 && a16(dq) && a16(dk) &&
        a16(dv)) {
        const float sl2 = scale * kLog2e;
        const dim3 gkv(static_cast<unsigned>((S + 127) / 128), static_cast<unsigned>(H), static_cast<unsigned>(B));
        const dim3 gq(static_cast<unsigned>((S + 127) / 128), static_cast<unsigned>(H), static_cast<unsigned>(B));
#define AIC_BWD_MFMA(HD_)                                                                                        \
    do {                                                                                                          \
        hipLaunchKernelGGL(attn_bwd_dkdv_mfma<HD_>, gkv, dim3(256), 0, s, static_cast<const bf16*>(q),            \
                           static_cast<const bf16*>(k), static_cast<const bf16*>(v), ld_qkv,                       \
                           static_cast<const bf16*>(dout), ld_o, lse, D, static_cast<bf16*>(dk),                   \
                           static_cast<bf16*>(dv), ld_d, static_cast<int>(H), static_cast<int>(S), sl2, scale,      \
                           causal ? 1 : 0);                                                                        \
        AIC_LAUNCH_CHECK("attn_bwd_dkdv_mfma");                                                                    \
        hipLaunchKernelGGL(attn_bwd_dq_mfma<HD_>, gq, dim3(256), 0, s, static_cast<const bf16*>(q),               \
                           static_cast<const bf16*>(k), static_cast<const bf16*>(v), ld_qkv,                       \
                           static_cast<const bf16*>(dout), ld_o, lse, D, static_cast<bf16*>(dq), ld_d,             \
                           static_cast<int>(H), static_cast<int>(S), sl2, scale, causal ? 1 : 0);                  \
        AIC_LAUNCH_CHECK("attn_bwd_dq_mfma");                                                                      \
    } while (0)
        if (hd == 128) AIC_BWD_MFMA(128);
        else AIC_BWD_MFMA(64);
#undef AIC_BWD_MFMA
        return;
    }
    if (dt == DType::Float32) bwd_simt<float>(q, k, v, ld_qkv, dout, ld_o, lse, D, dq, dk, dv, ld_d, B, H, S, hd, causal, scale, s);
    else bwd_simt<bf16>(q, k, v, ld_qkv, dout, ld_o, lse, D, dq, dk, dv, ld_d, B, H, S, hd, causal, scale, s);
}

}  // namespace aic::hip
