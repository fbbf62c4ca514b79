// Mixture-of-experts routing, dispatch and combine (the MoE FFN of MoETransformerBlock).
//
// Replaces MoERouter::route (src/nn/moe.cpp:33-129), which copies the gate logits to the
// host, partial-sorts every token there and copies indices, weights and counts back, and the
// dense dispatch of MoELayer::forward (moe.cpp:155-253), which runs every active expert on
// every token and multiplies by a zero gate for the tokens it does not own.  Here routing,
// counts and the auxiliary loss stay on the device, tokens are permuted into contiguous
// per-expert row blocks (a stable counting sort), each expert's SwiGLU runs only on its own
// rows, and the weighted combine gathers them back.  Nothing uses atomics: every reduction
// has a fixed order, so routing and gradients are bit-reproducible.
//
// Semantics shared with the reference (and the CPU oracle):
//   probs = softmax(logits) (max-shift, exp, sum, divide); top-k by logit, descending, ties to
//   the lower expert index (the reference's partial_sort leaves ties unspecified);
//   gates = probs * mask / (sum(probs * mask) + 1e-9) (moe.cpp:202-204);
//   aux = sum_e mean_t(probs[t, e]) * counts[e] * E * coef / (T * k) when coef > 0 and E > 1
//   (moe.cpp:84-101), the counts entering as constants.
#include <cstring>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

constexpr int kMaxE = 64;  // experts per layer handled by the per-token kernels
constexpr int kMaxK = 8;   // experts per token

// One thread per token: softmax over E, top-k selection, normalised gates of the selected.
// EM >= E bounds the per-token arrays at compile time (every loop unrolled to EM with an e < E
// guard and no runtime array index), so they stay in registers.
template <int EM>
__global__ __launch_bounds__(256) void moe_route_k(const float* __restrict__ logits, int T, int E, int k,
                                                   int64_t* __restrict__ idx, float* __restrict__ gsel,
                                                   float* __restrict__ probs, float* __restrict__ rweights) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const float* row = logits + static_cast<int64_t>(t) * E;
    float x[EM];
    float m = row[0];
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E) {
            x[e] = row[e];
            m = fmaxf(m, x[e]);
        }
    double s = 0.0;
    float p[EM];
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E) {
            p[e] = expf(x[e] - m);
            s += static_cast<double>(p[e]);
        }
    const float sf = static_cast<float>(s);
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E) {
            p[e] = p[e] / sf;
            probs[static_cast<int64_t>(t) * E + e] = p[e];
        }
    // selection: repeatedly the largest remaining logit, the lowest index among equals
    uint64_t used = 0;
    float selx[kMaxK], selp[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        if (j >= k) break;
        int best = -1;
        float bx = 0.0f, bp = 0.0f;
#pragma unroll
        for (int e = 0; e < EM; ++e)
            if (e < E && !((used >> e) & 1) && (best < 0 || x[e] > bx)) {
                best = e;
                bx = x[e];
                bp = p[e];
            }
        used |= 1ull << best;
        selx[j] = bx;
        selp[j] = bp;
        idx[static_cast<int64_t>(t) * k + j] = best;
    }
    double den = 0.0;
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E && ((used >> e) & 1)) den += static_cast<double>(p[e]);
    const float denf = static_cast<float>(den) + 1e-9f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
        if (j < k) gsel[static_cast<int64_t>(t) * k + j] = selp[j] / denf;
    if (rweights) {  // route()'s routing_weights: softmax over the selected logits (moe.cpp:67-77)
        const float mx = selx[0];
        float se = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxK; ++j)
            if (j < k) se += expf(selx[j] - mx);
#pragma unroll
        for (int j = 0; j < kMaxK; ++j)
            if (j < k) rweights[static_cast<int64_t>(t) * k + j] = expf(selx[j] - mx) / (se + 1e-9f);
    }
}

// Per-expert probability sums and counts of the tokens [blockIdx.x * kStatsTokens, + kStatsTokens):
// thread t takes one token for 8 experts at a time, the block's waves reduce with shuffles and
// their partials are added in wave order; part_p / part_c [block][E] (fixed order:
// deterministic).  Blocks of 256 tokens spread the pass over T / 256 CUs.
constexpr int kStatsTokens = 256;
__global__ __launch_bounds__(kStatsTokens) void moe_stats_k(const int64_t* __restrict__ idx,
                                                            const float* __restrict__ probs, int T, int E, int k,
                                                            double* __restrict__ part_p,
                                                            long long* __restrict__ part_c) {
    constexpr int NW = kStatsTokens / 64;
    __shared__ double sp[NW][kMaxE];
    __shared__ long long sc[NW][kMaxE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = static_cast<int>(blockIdx.x) * kStatsTokens + static_cast<int>(threadIdx.x);
    for (int e0 = 0; e0 < E; e0 += 8) {
        double a[8];
        long long c[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            a[u] = 0.0;
            c[u] = 0;
        }
        if (t < T) {
            const float* pr = probs + static_cast<int64_t>(t) * E + e0;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (e0 + u < E) a[u] = static_cast<double>(pr[u]);
            for (int j = 0; j < k; ++j) {
                const int64_t id = idx[static_cast<int64_t>(t) * k + j] - e0;
#pragma unroll
                for (int u = 0; u < 8; ++u) c[u] += id == u;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            for (int w = 32; w > 0; w >>= 1) {
                a[u] += __shfl_xor(a[u], w);
                c[u] += __shfl_xor(c[u], w);
            }
            if (lane == 0 && e0 + u < E) {
                sp[wave][e0 + u] = a[u];
                sc[wave][e0 + u] = c[u];
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < E) {
        double a = 0.0;
        long long c = 0;
        for (int w = 0; w < NW; ++w) {
            a += sp[w][threadIdx.x];
            c += sc[w][threadIdx.x];
        }
        part_p[static_cast<int64_t>(blockIdx.x) * E + threadIdx.x] = a;
        part_c[static_cast<int64_t>(blockIdx.x) * E + threadIdx.x] = c;
    }
}

// The block partials added in block order: counts, mean probabilities and the aux loss.
__global__ __launch_bounds__(64) void moe_stats_final_k(const double* __restrict__ part_p,
                                                        const long long* __restrict__ part_c, int nparts, int T,
                                                        int E, int k, float aux_coef, int64_t* __restrict__ counts,
                                                        float* __restrict__ mean_probs, float* __restrict__ aux) {
    __shared__ float mp_s[kMaxE];
    __shared__ long long cnt_s[kMaxE];
    if (threadIdx.x < E) {
        double a = 0.0;
        long long c = 0;
        int b = 0;
        // eight partials' loads in flight, added in block order
        for (; b + 8 <= nparts; b += 8) {
            double pa[8];
            long long pc[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                pa[u] = part_p[static_cast<int64_t>(b + u) * E + threadIdx.x];
                pc[u] = part_c[static_cast<int64_t>(b + u) * E + threadIdx.x];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                a += pa[u];
                c += pc[u];
            }
        }
        for (; b < nparts; ++b) {
            a += part_p[static_cast<int64_t>(b) * E + threadIdx.x];
            c += part_c[static_cast<int64_t>(b) * E + threadIdx.x];
        }
        mp_s[threadIdx.x] = static_cast<float>(a / static_cast<double>(T));
        cnt_s[threadIdx.x] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double a = 0.0;
        const float scale = (static_cast<float>(E) * aux_coef) / (static_cast<float>(T) * static_cast<float>(k));
        for (int e = 0; e < E; ++e) {
            if (mean_probs) mean_probs[e] = mp_s[e];
            counts[e] = cnt_s[e];
            a += static_cast<double>(mp_s[e] * (static_cast<float>(cnt_s[e]) * scale));
        }
        if (aux) *aux = (aux_coef > 0.0f && E > 1) ? static_cast<float>(a) : 0.0f;
    }
}

constexpr int kRowAlign = 64;  // each expert's row block starts at a multiple of 64 rows
__device__ __forceinline__ long long align_rows(long long n) { return (n + kRowAlign - 1) / kRowAlign * kRowAlign; }

constexpr int kPermRounds = 16;  // rounds of 1024 entries per pass of moe_permute_k

// One block per expert: stable positions of its (token, slot) entries in token order, in a
// row block that starts at offsets[e] (a multiple of 64; the block is padded to 64 rows).
// dst_row[t * k + j] = row of that entry; src_ent[row] = t * k + j, or -1 for a padding row.
__global__ __launch_bounds__(1024) void moe_permute_k(const int64_t* __restrict__ idx, const int64_t* __restrict__ counts,
                                                      int T, int k, int E, int max_rows,
                                                      int64_t* __restrict__ offsets, int* __restrict__ dst_row,
                                                      int* __restrict__ src_ent) {
    const int e = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __shared__ int wsum[kPermRounds][16], wpre[kPermRounds][16];
    __shared__ int base_s, start_s, total_s;
    if (threadIdx.x == 0) {
        long long off = 0;
        for (int i = 0; i < e; ++i) off += align_rows(counts[i]);
        base_s = static_cast<int>(off);
        start_s = static_cast<int>(off);
        if (e == 0) {
            long long o = 0;
            for (int i = 0; i < E; ++i) {
                offsets[i] = o;
                o += align_rows(counts[i]);
            }
            offsets[E] = o;
        }
    }
    __syncthreads();
    const int n = T * k;
    // passes of kPermRounds rounds of 1024 entries: all the rounds' loads in flight, a ballot
    // gives each hit its rank within its wave and round, and an exclusive scan of the
    // (round, wave) hit counts -- in entry order -- its offset, so the order stays the
    // entries' (token-major) order
    for (int c0 = 0; c0 < n; c0 += 1024 * kPermRounds) {
        bool hit[kPermRounds];
        unsigned long long m[kPermRounds];
#pragma unroll
        for (int r = 0; r < kPermRounds; ++r) {
            const int i = c0 + r * 1024 + static_cast<int>(threadIdx.x);
            hit[r] = i < n && idx[i] == e;
        }
#pragma unroll
        for (int r = 0; r < kPermRounds; ++r) {
            m[r] = __ballot(hit[r]);
            if (lane == 0) wsum[r][wave] = __popcll(m[r]);
        }
        __syncthreads();
        if (wave == 0) {  // exclusive scan of the kPermRounds x 16 counts, four per lane
            constexpr int PL = kPermRounds * 16 / 64;
            const int* cnt = &wsum[0][0];
            int v[PL], sum = 0;
#pragma unroll
            for (int q = 0; q < PL; ++q) {
                v[q] = cnt[lane * PL + q];
                sum += v[q];
            }
            int inc = sum;
#pragma unroll
            for (int w = 1; w < 64; w <<= 1) {
                const int t = __shfl_up(inc, w);
                if (lane >= w) inc += t;
            }
            int ex = inc - sum;
#pragma unroll
            for (int q = 0; q < PL; ++q) {
                (&wpre[0][0])[lane * PL + q] = ex;
                ex += v[q];
            }
            if (lane == 63) total_s = inc;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kPermRounds; ++r)
            if (hit[r]) {
                const int i = c0 + r * 1024 + static_cast<int>(threadIdx.x);
                const int row = base_s + wpre[r][wave] + __popcll(m[r] & ((1ull << lane) - 1ull));
                dst_row[i] = row;
                src_ent[row] = i;
            }
        __syncthreads();
        if (threadIdx.x == 0) base_s += total_s;
        __syncthreads();
    }
    // padding rows of this expert's block; the last expert also marks the rows after all
    // blocks (up to max_rows) as padding, so that every row of src_ent is defined
    const int end = e == E - 1 ? max_rows : start_s + static_cast<int>(align_rows(base_s - start_s));
    for (int r = base_s + static_cast<int>(threadIdx.x); r < end; r += 1024) src_ent[r] = -1;
}

// VN consecutive elements as floats, and back: VN = 8 is one 16-byte access for bf16 (two for
// fp32), VN = 1 the scalar form; the values and their rounding are the same either way.
template <int VN, typename T>
__device__ __forceinline__ void ldv(const T* p, float* v) {
    if constexpr (VN == 8 && std::is_same_v<T, bf16>) {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[2 * q] = __uint_as_float(w[q] << 16);
            v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
        }
    } else if constexpr (VN == 8) {
        const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        v[0] = ld(p, 0);
    }
}
template <int VN, typename T>
__device__ __forceinline__ void stv(T* p, const float* v) {
    if constexpr (VN == 8 && std::is_same_v<T, bf16>) {
        *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                  pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
    } else if constexpr (VN == 8) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        st(p, 0, v[0]);
    }
}

// xp[r, :] = x[token of entry src_ent[r], :], zero for padding rows
template <typename T, int VN>
__global__ __launch_bounds__(256) void moe_gather_k(const T* __restrict__ x, int64_t ldx, const int* __restrict__ src,
                                                    int k, int d, T* __restrict__ xp) {
    const int r = blockIdx.x;
    const int ent = src[r];
    T* o = xp + static_cast<int64_t>(r) * d;
    const T* sr = x + static_cast<int64_t>(ent < 0 ? 0 : ent / k) * ldx;
    // raw copies (VN elements of 16 bytes' worth, or one element)
    using V = std::conditional_t<VN == 1, T, uint4>;
    constexpr int PER = VN == 1 ? 1 : static_cast<int>(16 / sizeof(T));
    for (int c = threadIdx.x * PER; c < d; c += blockDim.x * PER)
        *reinterpret_cast<V*>(o + c) = ent < 0 ? V{} : *reinterpret_cast<const V*>(sr + c);
}

// The token's slots in increasing expert order (the order the reference accumulates experts).
__device__ __forceinline__ void slot_order(const int64_t* idx_t, int k, int* ord) {
    for (int j = 0; j < k; ++j) ord[j] = j;
    for (int a = 1; a < k; ++a)
        for (int b = a; b > 0 && idx_t[ord[b]] < idx_t[ord[b - 1]]; --b) {
            const int tmp = ord[b];
            ord[b] = ord[b - 1];
            ord[b - 1] = tmp;
        }
}

// out[t, :] = R[t, :] + sum over slots (increasing expert) of gsel[t, j] * ye[dst_row[t, j], :]
template <typename T, int VN>
__global__ __launch_bounds__(256) void moe_combine_k(const T* __restrict__ ye, const int64_t* __restrict__ idx,
                                                     const int* __restrict__ dst_row, const float* __restrict__ gsel,
                                                     int k, int d, const T* __restrict__ R, int64_t ldr,
                                                     T* __restrict__ out, int64_t ldo) {
    const int t = blockIdx.x;
    int ord[kMaxK], row[kMaxK];
    float gs[kMaxK];
    slot_order(idx + static_cast<int64_t>(t) * k, k, ord);
    for (int q = 0; q < k; ++q) {
        row[q] = dst_row[static_cast<int64_t>(t) * k + ord[q]];
        gs[q] = gsel[static_cast<int64_t>(t) * k + ord[q]];
    }
    for (int c = threadIdx.x * VN; c < d; c += blockDim.x * VN) {
        float y[VN], v[VN];
#pragma unroll
        for (int i = 0; i < VN; ++i) y[i] = 0.0f;
        for (int q = 0; q < k; ++q) {
            ldv<VN>(ye + static_cast<int64_t>(row[q]) * d + c, v);
#pragma unroll
            for (int i = 0; i < VN; ++i) y[i] += v[i] * gs[q];
        }
        if (R) {
            ldv<VN>(R + static_cast<int64_t>(t) * ldr + c, v);
#pragma unroll
            for (int i = 0; i < VN; ++i) y[i] = v[i] + y[i];
        } else {
#pragma unroll
            for (int i = 0; i < VN; ++i) y[i] = 0.0f + y[i];
        }
        stv<VN>(out + static_cast<int64_t>(t) * ldo + c, y);
    }
}

// Per expert row r (entry t * k + j): dye[r] = gsel[t, j] * dout[t] and
// dgsel[t, j] = sum_c dout[t, c] * ye[r, c] (double, fixed order); padding rows get dye = 0.
template <typename T, int VN>
__global__ __launch_bounds__(256) void moe_combine_bwd_k(const T* __restrict__ dout, int64_t ldo, const T* __restrict__ ye,
                                                         const int* __restrict__ src_ent, const float* __restrict__ gsel,
                                                         int k, int d, T* __restrict__ dye, float* __restrict__ dgsel) {
    const int r = blockIdx.x;
    const int ent = src_ent[r];
    T* dr = dye + static_cast<int64_t>(r) * d;
    if (ent < 0) {
        float z[VN];
#pragma unroll
        for (int i = 0; i < VN; ++i) z[i] = 0.0f;
        for (int c = threadIdx.x * VN; c < d; c += blockDim.x * VN) stv<VN>(dr + c, z);
        return;
    }
    const int t = ent / k;
    const float g = gsel[ent];
    __shared__ double red[256];
    double acc = 0.0;
    for (int c = threadIdx.x * VN; c < d; c += blockDim.x * VN) {
        float go[VN], yv[VN], o[VN];
        ldv<VN>(dout + static_cast<int64_t>(t) * ldo + c, go);
        ldv<VN>(ye + static_cast<int64_t>(r) * d + c, yv);
#pragma unroll
        for (int i = 0; i < VN; ++i) {
            acc += static_cast<double>(go[i] * yv[i]);
            o[i] = go[i] * g;
        }
        stv<VN>(dr + c, o);
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) dgsel[ent] = static_cast<float>(red[0]);
}

// dx[t, :] (+)= sum over slots (increasing expert) of dxp[dst_row[t, j], :]
template <typename T, int VN>
__global__ __launch_bounds__(256) void moe_scatter_k(const T* __restrict__ dxp, const int64_t* __restrict__ idx,
                                                     const int* __restrict__ dst_row, int k, int d, T* __restrict__ dx,
                                                     int64_t ldx, int accumulate, const float* __restrict__ dlog,
                                                     const T* __restrict__ wr, int E) {
    const int t = blockIdx.x;
    int ord[kMaxK], row[kMaxK];
    slot_order(idx + static_cast<int64_t>(t) * k, k, ord);
    for (int q = 0; q < k; ++q) row[q] = dst_row[static_cast<int64_t>(t) * k + ord[q]];
    for (int c = threadIdx.x * VN; c < d; c += blockDim.x * VN) {
        float sm[VN], v[VN];
#pragma unroll
        for (int i = 0; i < VN; ++i) sm[i] = 0.0f;
        for (int q = 0; q < k; ++q) {
            ldv<VN>(dxp + static_cast<int64_t>(row[q]) * d + c, v);
#pragma unroll
            for (int i = 0; i < VN; ++i) sm[i] += v[i];
        }
        if (dlog) {
            // the router's input gradient dlogits[t] . W_r, experts in order
            for (int e = 0; e < E; ++e) {
                const float g = dlog[static_cast<int64_t>(t) * E + e];
                ldv<VN>(wr + static_cast<int64_t>(e) * d + c, v);
#pragma unroll
                for (int i = 0; i < VN; ++i) sm[i] = fmaf(g, v[i], sm[i]);
            }
        }
        T* o = dx + static_cast<int64_t>(t) * ldx + c;
        if (accumulate) {
            ldv<VN>(o, v);
#pragma unroll
            for (int i = 0; i < VN; ++i) sm[i] = v[i] + sm[i];
        }
        stv<VN>(o, sm);
    }
}

// Router backward, one thread per token: gradient of the gates (normalisation and mask) and of
// the aux loss through both softmaxes into dlogits [T, E] (overwritten).  EM >= E as for
// moe_route_k.
template <int EM>
__global__ __launch_bounds__(256) void moe_router_bwd_k(const float* __restrict__ probs, const int64_t* __restrict__ idx,
                                                        const float* __restrict__ dgsel,
                                                        const int64_t* __restrict__ counts, int T, int E, int k,
                                                        float aux_coef, float daux, const float* __restrict__ daux_scale,
                                                        float* __restrict__ dlogits) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    if (daux_scale) daux *= *daux_scale;
    const float* pp = probs + static_cast<int64_t>(t) * E;
    float p[EM], dg[EM];
#pragma unroll
    for (int e = 0; e < EM; ++e) {
        p[e] = e < E ? pp[e] : 0.0f;
        dg[e] = 0.0f;
    }
    uint64_t used = 0;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        if (j >= k) break;
        const int sel = static_cast<int>(idx[static_cast<int64_t>(t) * k + j]);
        const float g = dgsel[static_cast<int64_t>(t) * k + j];
        used |= 1ull << sel;
#pragma unroll
        for (int e = 0; e < EM; ++e)
            if (e == sel) dg[e] = g;
    }
    double den = 0.0;
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E && ((used >> e) & 1)) den += static_cast<double>(p[e]);
    const float denf = static_cast<float>(den) + 1e-9f;
    double sb = 0.0;
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E && ((used >> e) & 1)) sb += static_cast<double>(-dg[e] * p[e] / (denf * denf));
    float dp[EM];
#pragma unroll
    for (int e = 0; e < EM; ++e) dp[e] = ((used >> e) & 1) ? (dg[e] / denf + static_cast<float>(sb)) : 0.0f;
    float dl[EM];
    double s = 0.0;
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E) s += static_cast<double>(dp[e]) * static_cast<double>(p[e]);
    float sf = static_cast<float>(s);
#pragma unroll
    for (int e = 0; e < EM; ++e) dl[e] = p[e] * (dp[e] - sf);
    if (aux_coef > 0.0f && E > 1) {
        const float fscale = (static_cast<float>(E) * aux_coef) / (static_cast<float>(T) * static_cast<float>(k));
        s = 0.0;
#pragma unroll
        for (int e = 0; e < EM; ++e)
            if (e < E) {
                dp[e] = (daux * (static_cast<float>(counts[e]) * fscale)) / static_cast<float>(T);
                s += static_cast<double>(dp[e]) * static_cast<double>(p[e]);
            }
        sf = static_cast<float>(s);
#pragma unroll
        for (int e = 0; e < EM; ++e) dl[e] += p[e] * (dp[e] - sf);
    }
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E) dlogits[static_cast<int64_t>(t) * E + e] = dl[e];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

void check_moe(int64_t T, int64_t E, int64_t k) {
    AIC_CHECK(T >= 1 && T < (1LL << 28), InvalidArgument, "moe: token count out of range");
    AIC_CHECK(E >= 1 && E <= kMaxE, InvalidArgument, "moe: experts must be in [1, ", kMaxE, "]");
    AIC_CHECK(k >= 1 && k <= kMaxK && k <= E, InvalidArgument, "moe: top_k must be in [1, min(E, ", kMaxK, ")]");
}

}  // namespace

void moe_route(const float* logits, int64_t T, int64_t E, int64_t k, float aux_coef, int64_t* idx, float* gsel,
               float* probs, float* rweights, int64_t* counts, float* mean_probs, float* aux, hipStream_t s) {
    check_moe(T, E, k);
    AIC_CHECK(logits && idx && gsel && probs && counts, InvalidArgument, "moe_route: null argument");
#define AIC_ROUTE(EM)                                                                                       \
    hipLaunchKernelGGL(moe_route_k<EM>, dim3(grid_for(T, 256)), dim3(256), 0, s, logits, static_cast<int>(T), \
                       static_cast<int>(E), static_cast<int>(k), idx, gsel, probs, rweights)
    if (E <= 8) AIC_ROUTE(8);
    else if (E <= 16) AIC_ROUTE(16);
    else if (E <= 32) AIC_ROUTE(32);
    else AIC_ROUTE(kMaxE);
#undef AIC_ROUTE
    AIC_LAUNCH_CHECK("moe_route");
    // statistics: kStatsTokens tokens per block, then the partials in block order
    const int nparts = static_cast<int>((T + kStatsTokens - 1) / kStatsTokens);
    double* part_p = static_cast<double*>(stream_scratch((sizeof(double) + sizeof(long long)) * nparts * E, s));
    long long* part_c = reinterpret_cast<long long*>(part_p + static_cast<int64_t>(nparts) * E);
    hipLaunchKernelGGL(moe_stats_k, dim3(static_cast<unsigned>(nparts)), dim3(kStatsTokens), 0, s, idx, probs,
                       static_cast<int>(T), static_cast<int>(E), static_cast<int>(k), part_p, part_c);
    AIC_LAUNCH_CHECK("moe_stats");
    hipLaunchKernelGGL(moe_stats_final_k, dim3(1), dim3(64), 0, s, part_p, part_c, nparts, static_cast<int>(T),
                       static_cast<int>(E), static_cast<int>(k), aux_coef, counts, mean_probs, aux);
    AIC_LAUNCH_CHECK("moe_stats_final");
}

int64_t moe_max_rows(int64_t T, int64_t E, int64_t k) { return T * k + E * (kRowAlign - 1); }

void moe_permute(const int64_t* idx, const int64_t* counts, int64_t T, int64_t k, int64_t E, int64_t* offsets,
                 int* dst_row, int* src_ent, hipStream_t s) {
    check_moe(T, E, k);
    AIC_CHECK(idx && counts && offsets && dst_row && src_ent, InvalidArgument, "moe_permute: null argument");
    AIC_CHECK(moe_max_rows(T, E, k) < (int64_t{1} << 31), InvalidArgument, "moe_permute: too many rows");
    hipLaunchKernelGGL(moe_permute_k, dim3(static_cast<unsigned>(E)), dim3(1024), 0, s, idx, counts,
                       static_cast<int>(T), static_cast<int>(k), static_cast<int>(E),
                       static_cast<int>(moe_max_rows(T, E, k)), offsets, dst_row, src_ent);
    AIC_LAUNCH_CHECK("moe_permute");
}

void moe_gather(const void* x, int64_t ldx, const int* src_ent, int64_t k, int64_t rows, int64_t d, void* xp, DType dt,
                hipStream_t s) {
    AIC_CHECK(rows >= 0 && d > 0 && ldx >= d && k >= 1, InvalidArgument, "moe_gather: bad shape");
    if (rows == 0) return;
    // 16-byte accesses when every row start is 16-byte aligned
    const bool v = d % 8 == 0 && ldx % 8 == 0 && aligned16(x) && aligned16(xp);
    const dim3 g(static_cast<unsigned>(rows)), b(v ? 128 : 256);
    if (dt == DType::BFloat16) {
        if (v) hipLaunchKernelGGL((moe_gather_k<bf16, 8>), g, b, 0, s, static_cast<const bf16*>(x), ldx, src_ent,
                                  static_cast<int>(k), static_cast<int>(d), static_cast<bf16*>(xp));
        else hipLaunchKernelGGL((moe_gather_k<bf16, 1>), g, b, 0, s, static_cast<const bf16*>(x), ldx, src_ent,
                                static_cast<int>(k), static_cast<int>(d), static_cast<bf16*>(xp));
    } else if (dt == DType::Float32) {
        if (v) hipLaunchKernelGGL((moe_gather_k<float, 8>), g, b, 0, s, static_cast<const float*>(x), ldx, src_ent,
                                  static_cast<int>(k), static_cast<int>(d), static_cast<float*>(xp));
        else hipLaunchKernelGGL((moe_gather_k<float, 1>), g, b, 0, s, static_cast<const float*>(x), ldx, src_ent,
                                static_cast<int>(k), static_cast<int>(d), static_cast<float*>(xp));
    } else {
        AIC_THROW(DTypeMismatch, "moe_gather: dtype must be f32 or bf16");
    }
    AIC_LAUNCH_CHECK("moe_gather");
}

void moe_combine(const void* ye, const int64_t* idx, const int* dst_row, const float* gsel, int64_t T, int64_t k,
                 int64_t d, const void* R, int64_t ldr, void* out, int64_t ldo, DType dt, hipStream_t s) {
    AIC_CHECK(T >= 0 && k >= 1 && k <= kMaxK && d > 0 && ldo >= d, InvalidArgument, "moe_combine: bad shape");
    if (T == 0) return;
    const bool v = d % 8 == 0 && ldo % 8 == 0 && aligned16(ye) && aligned16(out) &&
                   (!R || (ldr % 8 == 0 && aligned16(R)));
    const dim3 g(static_cast<unsigned>(T)), b(v ? 128 : 256);
#define AIC_COMBINE(TT, VN)                                                                                        \
    hipLaunchKernelGGL((moe_combine_k<TT, VN>), g, b, 0, s, static_cast<const TT*>(ye), idx, dst_row, gsel,       \
                       static_cast<int>(k), static_cast<int>(d), static_cast<const TT*>(R), ldr,                  \
                       static_cast<TT*>(out), ldo)
    if (dt == DType::BFloat16) {
        if (v) AIC_COMBINE(bf16, 8);
        else AIC_COMBINE(bf16, 1);
    } else if (dt == DType::Float32) {
        if (v) AIC_COMBINE(float, 8);
        else AIC_COMBINE(float, 1);
    } else {
        AIC_THROW(DTypeMismatch, "moe_combine: dtype must be f32 or bf16");
    }
#undef AIC_COMBINE
    AIC_LAUNCH_CHECK("moe_combine");
}

void moe_combine_bwd(const void* dout, int64_t ldo, const void* ye, const int* src_ent, const float* gsel, int64_t rows,
                     int64_t k, int64_t d, void* dye, float* dgsel, DType dt, hipStream_t s) {
    AIC_CHECK(rows >= 0 && k >= 1 && k <= kMaxK && d > 0 && ldo >= d, InvalidArgument, "moe_combine_bwd: bad shape");
    if (rows == 0) return;
    const bool v = d % 8 == 0 && ldo % 8 == 0 && aligned16(dout) && aligned16(ye) && aligned16(dye);
    const dim3 g(static_cast<unsigned>(rows)), b(v ? 128 : 256);
#define AIC_COMBINE_BWD(TT, VN)                                                                                    \
    hipLaunchKernelGGL((moe_combine_bwd_k<TT, VN>), g, b, 0, s, static_cast<const TT*>(dout), ldo,                \
                       static_cast<const TT*>(ye), src_ent, gsel, static_cast<int>(k), static_cast<int>(d),       \
                       static_cast<TT*>(dye), dgsel)
    if (dt == DType::BFloat16) {
        if (v) AIC_COMBINE_BWD(bf16, 8);
        else AIC_COMBINE_BWD(bf16, 1);
    } else if (dt == DType::Float32) {
        if (v) AIC_COMBINE_BWD(float, 8);
        else AIC_COMBINE_BWD(float, 1);
    } else {
        AIC_THROW(DTypeMismatch, "moe_combine_bwd: dtype must be f32 or bf16");
    }
#undef AIC_COMBINE_BWD
    AIC_LAUNCH_CHECK("moe_combine_bwd");
}

void moe_scatter(const void* dxp, const int64_t* idx, const int* dst_row, int64_t T, int64_t k, int64_t d, void* dx,
                 int64_t ldx, bool accumulate, DType dt, hipStream_t s, const float* router_dlogits,
                 const void* router_w, int64_t E) {
    AIC_CHECK(T >= 0 && k >= 1 && k <= kMaxK && d > 0 && ldx >= d, InvalidArgument, "moe_scatter: bad shape");
    AIC_CHECK(!router_dlogits || (router_w && E >= 1 && E <= kMaxE), InvalidArgument, "moe_scatter: bad router term");
    if (T == 0) return;
    const bool v = d % 8 == 0 && ldx % 8 == 0 && aligned16(dxp) && aligned16(dx) && (!router_w || aligned16(router_w));
    const dim3 g(static_cast<unsigned>(T)), b(v ? 128 : 256);
#define AIC_SCATTER(TT, VN)                                                                                        \
    hipLaunchKernelGGL((moe_scatter_k<TT, VN>), g, b, 0, s, static_cast<const TT*>(dxp), idx, dst_row,             \
                       static_cast<int>(k), static_cast<int>(d), static_cast<TT*>(dx), ldx, accumulate ? 1 : 0,    \
                       router_dlogits, static_cast<const TT*>(router_w), static_cast<int>(E))
    if (dt == DType::BFloat16) {
        if (v) AIC_SCATTER(bf16, 8);
        else AIC_SCATTER(bf16, 1);
    } else if (dt == DType::Float32) {
        if (v) AIC_SCATTER(float, 8);
        else AIC_SCATTER(float, 1);
    } else {
        AIC_THROW(DTypeMismatch, "moe_scatter: dtype must be f32 or bf16");
    }
#undef AIC_SCATTER
    AIC_LAUNCH_CHECK("moe_scatter");
}

void moe_router_bwd(const float* probs, const int64_t* idx, const float* dgsel, const int64_t* counts, int64_t T,
                    int64_t E, int64_t k, float aux_coef, float daux, const float* daux_scale, float* dlogits,
                    hipStream_t s) {
    check_moe(T, E, k);
#define AIC_ROUTER_BWD(EM)                                                                                 \
    hipLaunchKernelGGL(moe_router_bwd_k<EM>, dim3(grid_for(T, 256)), dim3(256), 0, s, probs, idx, dgsel, counts, \
                       static_cast<int>(T), static_cast<int>(E), static_cast<int>(k), aux_coef, daux, daux_scale,  \
                       dlogits)
    if (E <= 8) AIC_ROUTER_BWD(8);
    else if (E <= 16) AIC_ROUTER_BWD(16);
    else if (E <= 32) AIC_ROUTER_BWD(32);
    else AIC_ROUTER_BWD(kMaxE);
#undef AIC_ROUTER_BWD
    AIC_LAUNCH_CHECK("moe_router_bwd");
}

namespace {
__global__ void moe_aux_total_k(const float* __restrict__ aux, int L, float* __restrict__ loss, float* __restrict__ total) {
    float t = aux[0];
    for (int l = 1; l < L; ++l) t = t + aux[l];  // add(add(aux_0, aux_1), ...) in layer order
    *total = t;
    *loss = *loss + t;
}
}  // namespace

void moe_aux_total(const float* aux, int64_t L, float* loss, float* total, hipStream_t s) {
    AIC_CHECK(L >= 1 && aux && loss && total, InvalidArgument, "moe_aux_total: bad arguments");
    hipLaunchKernelGGL(moe_aux_total_k, dim3(1), dim3(1), 0, s, aux, static_cast<int>(L), loss, total);
    AIC_LAUNCH_CHECK("moe_aux_total");
}

}  // namespace aic::hip
