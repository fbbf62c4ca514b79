// LoRA adapter products as single passes over the large operand.
//
// A LoRA projection (LoRALinear, src/nn/lora.cpp:75-93, differentiated by the reference's
// autograd) needs, besides the frozen base product, products whose result has only r (the
// rank) columns:
//   forward   xs  = s x A^T                  [T, r]   (a reduction over the input width)
//   backward  dB  = dy^T xs                  [out, r] (a reduction over the tokens)
//             dxa = s dy B                   [T, r]   (a reduction over the output width)
//             dA  = dxa^T x                  [r, in]  (a reduction over the tokens)
// As GEMMs these are tall-skinny: an MFMA tile of 128 or 256 columns is mostly padding, and
// the token reductions need split-K and a reduction pass.  Their cost is reading the large
// operand (x or dy: T x width bf16) from HBM.  Here one kernel streams that operand once
// through LDS in stages of 64 rows x 256 columns and forms, per stage,
//   P1  out1[t, j] += sum_n Y[t, n] W(n, j)     (the stage's rows against W's rows n)
//   P2  out2[n, j] += sum_t Y[t, n] Z[t, j]     (the stage's columns against Z's rows t)
// with v_mfma_f32_16x16x32_bf16: P1 reads Y rows (ds_read_b128), P2 reads Y columns from the
// same tile with ds_read_b64_tr_b16, so dB and dxa of a projection come from one pass over dy.
// Y's columns may be split into segments (q, k, v stacked, or gate and up): segment g of
// n_seg columns pairs with columns [g r_seg, (g+1) r_seg) of Z and of out1.
// Blocks cover 64..512 rows x 256 columns (P2) or 64 rows x several chunks (P1 only); partial
// sums over column groups (P1) or row blocks (P2) go to scratch in fp32 and a second kernel
// adds them in a fixed order, so the results are deterministic (no atomics).
#include "common.hpp"
#include "kernels.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::hip {

namespace {

constexpr int kSub = 64;            // rows of a stage
constexpr int kChunk = 256;         // columns of a stage
constexpr int kYPitch = kChunk + 8; // bf16 per LDS row of the Y stage (16 bytes of padding)
constexpr int kZPitch = kSub + 8;   // bf16 per LDS row of Z^T (t along the row)

struct SkinnyParams {
    const bf16* Y;
    int64_t ldy;
    int T, N, n_seg, r_seg;
    // P1
    const bf16* W;
    int64_t w_n, w_j;    // W(n, j) = W[n w_n + j w_j]; w_j == 1 (rows of r_seg) or w_n == 1
    float* p1;           // partials [groups][T][r_seg], or null: direct bf16 output
    bf16* out1;
    int64_t ldo1;
    float scale;
    // P2
    const bf16* Z;
    int64_t ldz;
    float* p2;           // partials [row blocks][N][r_seg], or null: direct fp32 output
    float* out2;
    int64_t o2n, o2j;
    int accumulate;
    int tt;              // rows per block (a multiple of 64)
    int cpb;             // 256-column chunks per block
};

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Transposed fragment of the Y stage for the P2 A operand: lane (g = lane / 16, i = lane % 16)
// receives column c0 + i at rows r0 + 8 g + 0..7.  Each ds_read_b64_tr_b16 hands lane i of a
// 16-lane group slot q the element i % 4 of the 4 values that source lane 4 q + i / 4 of the
// group addressed, so source lane s addresses row (r0 + 8 g + 4 u + s / 4), columns
// c0 + 4 (s % 4) .. +3, for the two halves u = 0, 1.
__device__ __forceinline__ bf16x8 ytr(const bf16* ys, int r0, int c0) {
    const int lane = threadIdx.x & 63, g = lane >> 4, s = lane & 15;
    const bf16* p0 = ys + (r0 + 8 * g + (s >> 2)) * kYPitch + c0 + 4 * (s & 3);
    const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p0));
    const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p0 + 4 * kYPitch));
    const u32x2 x = __builtin_bit_cast(u32x2, a), y = __builtin_bit_cast(u32x2, b);
    return __builtin_bit_cast(bf16x8, make_uint4(x.x, x.y, y.x, y.y));
}

template <int RB, bool P1, bool P2>
__global__ __launch_bounds__(256, 2) void lora_skinny_k(SkinnyParams p) {
    constexpr int R = 16 * RB;
    constexpr int YCH = kSub * kChunk / 8 / 256;        // 16-byte Y chunks per thread per stage (8)
    constexpr int WCH = (P1 ? R * kChunk / 8 + 255 : 0) / 256;  // W^T chunks per thread
    constexpr int ZCH = (P2 ? kSub * R / 8 + 255 : 0) / 256;    // Z chunks per thread
    __shared__ __align__(16) bf16 ys[kSub * kYPitch];
    __shared__ __align__(16) bf16 wt[P1 ? R * kYPitch : 8];
    __shared__ __align__(16) bf16 zt[P2 ? R * kZPitch : 8];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, i = lane & 15;
    const int n_base = blockIdx.x * p.cpb * kChunk;  // first column of the block
    const int seg = n_base / p.n_seg;
    const int t_base = blockIdx.y * p.tt;
    const int nsub = min(p.tt, p.T - t_base + kSub - 1) / kSub;
    const int nstage = nsub * p.cpb;

    uint4 yr[YCH];
    uint4 wr[WCH > 0 ? WCH : 1];
    uint4 zr[ZCH > 0 ? ZCH : 1];
    auto load = [&](int st) {
        const int sub = st / p.cpb, c = st % p.cpb;
        const int t0 = t_base + sub * kSub, n0 = n_base + c * kChunk;
#pragma unroll
        for (int k = 0; k < YCH; ++k) {
            const int e = tid + 256 * k, row = e >> 5, col = (e & 31) * 8;
            yr[k] = t0 + row < p.T ? *reinterpret_cast<const uint4*>(p.Y + (int64_t)(t0 + row) * p.ldy + n0 + col)
                                   : make_uint4(0, 0, 0, 0);
        }
        if constexpr (P1) {
            if (p.cpb > 1 || st == 0) {
#pragma unroll
                for (int k = 0; k < WCH; ++k) {
                    const int e = tid + 256 * k;
                    if (e < R * kChunk / 8) {
                        if (p.w_j == 1) {  // rows n of r_seg contiguous j: chunk = (n, 8 j's)
                            const int n = e / RB / 2, j8 = (e % (2 * RB)) * 8;
                            wr[k] = *reinterpret_cast<const uint4*>(p.W + (int64_t)(n0 + n) * p.w_n + j8);
                        } else {           // rows j of contiguous n: chunk = (j, 8 n's)
                            const int j = e >> 5, n8 = (e & 31) * 8;
                            wr[k] = *reinterpret_cast<const uint4*>(p.W + (int64_t)j * p.w_j + n0 + n8);
                        }
                    }
                }
            }
        }
        if constexpr (P2) {
            if (c == 0) {
#pragma unroll
                for (int k = 0; k < ZCH; ++k) {
                    const int e = tid + 256 * k, row = e / (2 * RB), j8 = (e % (2 * RB)) * 8;
                    if (e < kSub * R / 8)
                        zr[k] = t0 + row < p.T ? *reinterpret_cast<const uint4*>(p.Z + (int64_t)(t0 + row) * p.ldz +
                                                                                 seg * p.r_seg + j8)
                                               : make_uint4(0, 0, 0, 0);
                }
            }
        }
    };
    auto store = [&](int st) {
        const int c = st % p.cpb;
#pragma unroll
        for (int k = 0; k < YCH; ++k) {
            const int e = tid + 256 * k, row = e >> 5, col = (e & 31) * 8;
            *reinterpret_cast<uint4*>(ys + row * kYPitch + col) = yr[k];
        }
        if constexpr (P1) {
            if (p.cpb > 1 || st == 0) {
#pragma unroll
                for (int k = 0; k < WCH; ++k) {
                    const int e = tid + 256 * k;
                    if (e < R * kChunk / 8) {
                        if (p.w_j == 1) {
                            const int n = e / RB / 2, j8 = (e % (2 * RB)) * 8;
                            const bf16x8 v = __builtin_bit_cast(bf16x8, wr[k]);
#pragma unroll
                            for (int q = 0; q < 8; ++q) wt[(j8 + q) * kYPitch + n] = v[q];
                        } else {
                            const int j = e >> 5, n8 = (e & 31) * 8;
                            *reinterpret_cast<uint4*>(wt + j * kYPitch + n8) = wr[k];
                        }
                    }
                }
            }
        }
        if constexpr (P2) {
            if (c == 0) {
#pragma unroll
                for (int k = 0; k < ZCH; ++k) {
                    const int e = tid + 256 * k, row = e / (2 * RB), j8 = (e % (2 * RB)) * 8;
                    if (e < kSub * R / 8) {
                        const bf16x8 v = __builtin_bit_cast(bf16x8, zr[k]);
#pragma unroll
                        for (int q = 0; q < 8; ++q) zt[(j8 + q) * kZPitch + row] = v[q];
                    }
                }
            }
        }
    };

    f32x4 acc1[RB];
    f32x4 acc2[4][RB];
#pragma unroll
    for (int cb = 0; cb < RB; ++cb) {
        acc1[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) acc2[mb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    load(0);
    for (int st = 0; st < nstage; ++st) {
        const int sub = st / p.cpb, c = st % p.cpb;
        __syncthreads();  // the previous stage's reads of the LDS tiles are done
        store(st);
        __syncthreads();
        if (st + 1 < nstage) load(st + 1);  // in flight while this stage computes
        if constexpr (P1) {
            // wave w: rows 16 w .. +15 of the stage against all R columns, k over the chunk
#pragma unroll
            for (int ks = 0; ks < kChunk / 32; ++ks) {
                const bf16x8 a = *reinterpret_cast<const bf16x8*>(ys + (16 * w + i) * kYPitch + 32 * ks + 8 * g);
#pragma unroll
                for (int cb = 0; cb < RB; ++cb) {
                    const bf16x8 b = *reinterpret_cast<const bf16x8*>(wt + (16 * cb + i) * kYPitch + 32 * ks + 8 * g);
                    acc1[cb] = mfma16(a, b, acc1[cb]);
                }
            }
            if (c == p.cpb - 1) {
                // D of a 16x16 tile: lane (g, i) holds rows 4 g + v, column i
                const int grp = blockIdx.x, t_row = t_base + sub * kSub + 16 * w + 4 * g;
#pragma unroll
                for (int cb = 0; cb < RB; ++cb) {
                    const int j = 16 * cb + i;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int t = t_row + v;
                        if (t < p.T && j < p.r_seg) {
                            if (p.p1)
                                p.p1[((int64_t)grp * p.T + t) * p.r_seg + j] = acc1[cb][v];
                            else
                                p.out1[(int64_t)t * p.ldo1 + seg * p.r_seg + j] = f2bf(p.scale * acc1[cb][v]);
                        }
                    }
                    acc1[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
        }
        if constexpr (P2) {
            // wave w: columns 64 w .. +63 of the chunk (four 16-column tiles) against all R
#pragma unroll
            for (int ks = 0; ks < kSub / 32; ++ks) {
                bf16x8 b[RB];
#pragma unroll
                for (int cb = 0; cb < RB; ++cb)
                    b[cb] = *reinterpret_cast<const bf16x8*>(zt + (16 * cb + i) * kZPitch + 32 * ks + 8 * g);
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    const bf16x8 a = ytr(ys, 32 * ks, 64 * w + 16 * mb);
#pragma unroll
                    for (int cb = 0; cb < RB; ++cb) acc2[mb][cb] = mfma16(a, b[cb], acc2[mb][cb]);
                }
            }
        }
    }
    if constexpr (P2) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int cb = 0; cb < RB; ++cb) {
                const int j = 16 * cb + i;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int n = n_base + 64 * w + 16 * mb + 4 * g + v;
                    if (j < p.r_seg) {
                        if (p.p2) {
                            p.p2[((int64_t)blockIdx.y * p.N + n) * p.r_seg + j] = acc2[mb][cb][v];
                        } else {
                            float* o = p.out2 + (int64_t)n * p.o2n + (int64_t)j * p.o2j;
                            *o = p.accumulate ? *o + acc2[mb][cb][v] : acc2[mb][cb][v];
                        }
                    }
                }
            }
    }
}

// The forward product alone (out1 = bf16(scale * Y W), one segment, W(n, j) = W[j w_j + n]: the
// adapters' A [R, in]) without partial sums: a block owns 32 rows of Y and the whole width; wave
// w takes the 256-column chunks w, w + 8, ... for all 32 rows, as two 16-row MFMA tiles sharing
// each A fragment.  Both MFMA operands come straight from global memory in fragment layout -- a
// lane's 16 bytes of a Y row are one aligned quarter of a 64-byte segment that the 16 lanes of its
// row group read together, A's from L2 -- so nothing is staged in LDS; the eight waves' partial
// tiles are added in LDS in wave order at the end.
template <int RB>
__global__ __launch_bounds__(512) void lora_xa_k(SkinnyParams p) {
    constexpr int R = 16 * RB;
    __shared__ float red[8][32][R];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, i = lane & 15;
    const int t0 = blockIdx.x * 32;
    const bool ok0 = t0 + i < p.T, ok1 = t0 + 16 + i < p.T;
    const bf16* y0 = p.Y + (int64_t)(ok0 ? t0 + i : 0) * p.ldy + 8 * g;
    const bf16* y1 = p.Y + (int64_t)(ok1 ? t0 + 16 + i : 0) * p.ldy + 8 * g;
    const bf16* wcol[RB];
#pragma unroll
    for (int cb = 0; cb < RB; ++cb) wcol[cb] = p.W + (int64_t)(16 * cb + i) * p.w_j + 8 * g;
    f32x4 acc0[RB], acc1[RB];
#pragma unroll
    for (int cb = 0; cb < RB; ++cb) acc0[cb] = acc1[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int chunks = p.N / kChunk;
    for (int c = w; c < chunks; c += 8) {
        const int n0 = c * kChunk;
        bf16x8 a0[8], a1[8], b[8][RB];
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            a0[ks] = ok0 ? *reinterpret_cast<const bf16x8*>(y0 + n0 + 32 * ks) : bf16x8{};
            a1[ks] = ok1 ? *reinterpret_cast<const bf16x8*>(y1 + n0 + 32 * ks) : bf16x8{};
#pragma unroll
            for (int cb = 0; cb < RB; ++cb) b[ks][cb] = *reinterpret_cast<const bf16x8*>(wcol[cb] + n0 + 32 * ks);
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
#pragma unroll
            for (int cb = 0; cb < RB; ++cb) {
                acc0[cb] = mfma16(a0[ks], b[ks][cb], acc0[cb]);
                acc1[cb] = mfma16(a1[ks], b[ks][cb], acc1[cb]);
            }
    }
    // D of a 16x16 tile: lane (g, i) holds rows 4 g + v, column i
#pragma unroll
    for (int cb = 0; cb < RB; ++cb)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            red[w][4 * g + v][16 * cb + i] = acc0[cb][v];
            red[w][16 + 4 * g + v][16 * cb + i] = acc1[cb][v];
        }
    __syncthreads();
    for (int e = tid; e < 32 * R; e += 512) {
        const int row = e / R, j = e % R;
        if (t0 + row < p.T) {
            float sum = red[0][row][j];
#pragma unroll
            for (int k = 1; k < 8; ++k) sum += red[k][row][j];
            p.out1[(int64_t)(t0 + row) * p.ldo1 + j] = f2bf(p.scale * sum);
        }
    }
}

// Fixed-order sums of the partials, four consecutive j per thread (r_seg % 16 == 0).  Threads
// [0, n1): out1[t, g r_seg + j] = bf16(scale * sum over the column groups of segment g); threads
// [n1, n1 + n2): out2(n, j) = sum over the row blocks.
__global__ __launch_bounds__(256) void lora_reduce_k(SkinnyParams p, int groups_per_seg, int segs, int row_blocks) {
    const int q4 = p.r_seg / 4;
    const int64_t n1 = p.p1 ? (int64_t)p.T * segs * q4 : 0;
    const int64_t n2 = p.p2 ? (int64_t)p.N * q4 : 0;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < n1) {
        const int j = 4 * (idx % q4);
        const int64_t rest = idx / q4;
        const int sg = rest % segs;
        const int64_t t = rest / segs;
        const float* src = p.p1 + ((int64_t)sg * groups_per_seg * p.T + t) * p.r_seg + j;
        const int64_t stride = (int64_t)p.T * p.r_seg;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
        for (int q = 0; q < groups_per_seg; ++q) {
            const float4 v = *reinterpret_cast<const float4*>(src + q * stride);
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
        *reinterpret_cast<uint2*>(p.out1 + t * p.ldo1 + sg * p.r_seg + j) =
            make_uint2(pack_bf16x2(p.scale * acc.x, p.scale * acc.y), pack_bf16x2(p.scale * acc.z, p.scale * acc.w));
    } else if (idx < n1 + n2) {
        const int64_t e = idx - n1;
        const int j = 4 * (e % q4);
        const int64_t n = e / q4;
        const float* src = p.p2 + n * p.r_seg + j;
        const int64_t stride = (int64_t)p.N * p.r_seg;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
        for (int q = 0; q < row_blocks; ++q) {
            const float4 v = *reinterpret_cast<const float4*>(src + q * stride);
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
        const float a[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float* o = p.out2 + n * p.o2n + (int64_t)(j + u) * p.o2j;
            *o = p.accumulate ? *o + a[u] : a[u];
        }
    }
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// Compute units of the current device (cached per device): sizes the grid.
int cus_of_device() {
    static int cus[64] = {};
    int dev = 0;
    AIC_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        AIC_HIP_CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        cus[dev] = n > 0 ? n : 256;
    }
    return cus[dev];
}

}  // namespace

bool lora_skinny_ok(const LoraSkinny& q) {
    const bool p1 = q.out1 != nullptr, p2 = q.out2 != nullptr;
    if (!(p1 || p2) || !q.Y || q.T <= 0 || q.N <= 0 || q.T >= (int64_t{1} << 30)) return false;
    if (q.n_seg <= 0 || q.n_seg % kChunk != 0 || q.N % q.n_seg != 0 || q.N >= (int64_t{1} << 30)) return false;
    if (q.r_seg != 16 && q.r_seg != 32 && q.r_seg != 48) return false;
    if (q.ldy < q.N || q.ldy % 8 != 0 || !aligned16(q.Y)) return false;
    if (p1) {
        if (!q.W || !aligned16(q.W) || q.ldo1 < (q.N / q.n_seg) * q.r_seg) return false;
        if (q.ldo1 % 4 != 0 || (reinterpret_cast<uintptr_t>(q.out1) & 7u) != 0) return false;  // 8-byte stores
        const bool nj = q.w_j == 1 && q.w_n >= q.r_seg && q.w_n % 8 == 0;
        const bool jn = q.w_n == 1 && q.w_j >= q.n_seg && q.w_j % 8 == 0;
        if (!nj && !jn) return false;
    }
    if (p2) {
        if (!q.Z || !aligned16(q.Z) || q.ldz % 8 != 0 || q.ldz < (q.N / q.n_seg) * q.r_seg) return false;
    }
    return true;
}

void lora_skinny(const LoraSkinny& q, hipStream_t s) {
    AIC_CHECK(lora_skinny_ok(q), InvalidArgument, "lora_skinny: shape or layout outside the kernel's forms");
    const bool p1 = q.out1 != nullptr, p2 = q.out2 != nullptr;
    const int RB = static_cast<int>(q.r_seg / 16);
    const int64_t chunks = q.N / kChunk, cps = q.n_seg / kChunk;  // chunks in total and per segment
    const int cus = cus_of_device();
    SkinnyParams p{};
    p.Y = static_cast<const bf16*>(q.Y);
    p.ldy = q.ldy;
    p.T = static_cast<int>(q.T);
    p.N = static_cast<int>(q.N);
    p.n_seg = static_cast<int>(q.n_seg);
    p.r_seg = static_cast<int>(q.r_seg);
    p.W = static_cast<const bf16*>(q.W);
    p.w_n = q.w_n;
    p.w_j = q.w_j;
    p.out1 = static_cast<bf16*>(q.out1);
    p.ldo1 = q.ldo1;
    p.scale = q.scale;
    p.Z = static_cast<const bf16*>(q.Z);
    p.ldz = q.ldz;
    p.out2 = q.out2;
    p.o2n = q.o2n;
    p.o2j = q.o2j;
    p.accumulate = q.accumulate ? 1 : 0;
    const int64_t sub_rows = (q.T + kSub - 1) / kSub;
    if (p1 && !p2 && q.w_n == 1 && q.n_seg == q.N) {
        // the forward x A^T: 32 rows per block, no partial sums
        const dim3 grid(static_cast<unsigned>((q.T + 31) / 32));
        if (RB == 1) hipLaunchKernelGGL((lora_xa_k<1>), grid, dim3(512), 0, s, p);
        else if (RB == 2) hipLaunchKernelGGL((lora_xa_k<2>), grid, dim3(512), 0, s, p);
        else hipLaunchKernelGGL((lora_xa_k<3>), grid, dim3(512), 0, s, p);
        AIC_LAUNCH_CHECK("lora_xa");
        return;
    }
    if (p2) {
        // one chunk per block; rows per block halved from 512 until the grid covers the CUs
        p.cpb = 1;
        int64_t tt = 512;
        while (tt > kSub && chunks * ((q.T + tt - 1) / tt) < cus) tt /= 2;
        p.tt = static_cast<int>(tt);
    } else {
        // 64 rows per block; a segment's chunks split between blocks until the grid covers the CUs
        p.tt = kSub;
        int64_t cpb = cps;
        while (cpb % 2 == 0 && sub_rows * (chunks / cpb) < cus) cpb /= 2;
        p.cpb = static_cast<int>(cpb);
    }
    const int64_t groups = chunks / p.cpb, row_blocks = (q.T + p.tt - 1) / p.tt;
    const int64_t gps = cps / p.cpb, segs = q.N / q.n_seg;
    if (p1 && gps > 1) p.p1 = static_cast<float*>(stream_scratch(sizeof(float) * groups * q.T * q.r_seg, s, 2));
    if (p2 && row_blocks > 1)
        p.p2 = static_cast<float*>(stream_scratch(sizeof(float) * row_blocks * q.N * q.r_seg, s, 3));
    const dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>(row_blocks));
#define AIC_LORA(RB_, P1_, P2_) hipLaunchKernelGGL((lora_skinny_k<RB_, P1_, P2_>), grid, dim3(256), 0, s, p)
#define AIC_LORA_RB(P1_, P2_) \
    do {                      \
        if (RB == 1)          \
            AIC_LORA(1, P1_, P2_); \
        else if (RB == 2)     \
            AIC_LORA(2, P1_, P2_); \
        else                  \
            AIC_LORA(3, P1_, P2_); \
    } while (0)
    if (p1 && p2) AIC_LORA_RB(true, true);
    else if (p1) AIC_LORA_RB(true, false);
    else AIC_LORA_RB(false, true);
#undef AIC_LORA_RB
#undef AIC_LORA
    AIC_LAUNCH_CHECK("lora_skinny");
    if (p.p1 || p.p2) {
        const int64_t n = (p.p1 ? q.T * segs * q.r_seg / 4 : 0) + (p.p2 ? q.N * q.r_seg / 4 : 0);
        hipLaunchKernelGGL(lora_reduce_k, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, p,
                           static_cast<int>(gps), static_cast<int>(segs), static_cast<int>(row_blocks));
        AIC_LAUNCH_CHECK("lora_reduce");
    }
}

}  // namespace aic::hip
