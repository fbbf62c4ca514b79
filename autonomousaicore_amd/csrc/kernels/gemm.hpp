// Host interface of the GEMM kernels (see gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../runtime/dtype.hpp"

namespace aic::hip {

// Row-major C[M,N] = alpha * op(A) . op(B) + beta * C + R, fp32 accumulation.
//   op(A) is M x K: A[m*lda + k], or A[k*lda + m] when transA.
//   op(B) is K x N: B[k*ldb + n], or B[n*ldb + k] when transB.
// Linear forward y = x W^T is (transA=0, transB=1); dx = dy W is (0, 0); dW = dy^T x is (1, 0).
// R (optional, same dtype as C, leading dimension ldr) is added after scaling; beta == 0
// never reads C.
struct GemmArgs {
    int transA = 0, transB = 0;
    int64_t M = 0, N = 0, K = 0;
    float alpha = 1.0f, beta = 0.0f;
    const void* A = nullptr;
    int64_t lda = 0;
    const void* B = nullptr;
    int64_t ldb = 0;
    void* C = nullptr;
    int64_t ldc = 0;
    const void* R = nullptr;
    int64_t ldr = 0;
    DType ab = DType::BFloat16;
    DType c = DType::BFloat16;
    // Optional low-rank term (the LoRA path), added to the product before scaling:
    //   C = alpha * (op(A) op(B) + X2 Y2^T) + beta * C + R
    // X2 [M, r2] row-major (ldx2; with seg_n > 0, output columns [s seg_n, (s+1) seg_n) take
    // the X2 columns [s r2, (s+1) r2)); Y2 [N, r2] row-major (ldy2), or [r2, N] when
    // y2_kmajor.  Same dtype as A and B.
    const void* X2 = nullptr;
    const void* Y2 = nullptr;
    int64_t ldx2 = 0, ldy2 = 0, r2 = 0, seg_n = 0;
    int y2_kmajor = 0;
    // Optional INT4 B operand (the QLoRA base weight; B is then ignored).  The weight is
    // contiguous with row length ldb: W [N][ldb] when transB (the Linear forward x W^T), W [K][ldb]
    // otherwise (the input gradient dy W).  Bq holds its symmetric INT4 values two per byte
    // (element 2i in the low nibble of byte i), Bscale one scale (scale_t: f16 or f32) per `group`
    // consecutive elements of its flat row-major index; op(B) = q * scale, rounded to bf16 as
    // the standalone dequantization does, inside the kernel (gemm_q4_eligible lists the shapes).
    const uint8_t* Bq = nullptr;
    const void* Bscale = nullptr;
    DType scale_t = DType::Float16;
    int64_t group = 0;
    // Optional rotary embedding of the output (the attention projection's q and k): columns
    // [0, rope_cols) of C are heads of rope_hd values that leave rotated by the half-split RoPE
    // (rope(), RotaryPositionEmbedding::forward) at position rope_start + row % rope_seq, with
    // rope_cos / rope_sin the [positions][rope_hd / 2] tables.  Done in the GEMM's epilogue for
    // bf16 output on full 256x256 tiles with rope_hd 128; otherwise rope() runs after it.
    const float* rope_cos = nullptr;
    const float* rope_sin = nullptr;
    int64_t rope_cols = 0, rope_hd = 0, rope_seq = 0, rope_start = 0;
    // Optional SwiGLU activation of a gate/up product (N == 2 glu_f: C's columns [0, glu_f) are
    // the gate, [glu_f, 2 glu_f) the up projection): the product also writes
    // glu_out[row][j] = silu(C[row][j]) * C[row][glu_f + j] (bf16, leading dimension ld_glu) as
    // swiglu_fwd does.  In the epilogue for bf16 x W^T on full 256x256 tiles that pair 128 gate
    // with the matching 128 up columns (glu_f % 128 == 0); otherwise swiglu_fwd runs after it.
    int64_t glu_f = 0;
    void* glu_out = nullptr;
    int64_t ld_glu = 0;
    // Optional SwiGLU backward fed by the product (the down projection's input gradient
    // dh = dy W_d, [M, N = f]): with g = dglu_gu[row][j], u = dglu_gu[row][N + j] (leading
    // dimension dglu_ld) and dh the bf16 product, dglu_out[row][j] = dh u silu'(g) and
    // dglu_out[row][N + j] = dh silu(g) (swiglu_bwd's arithmetic).  In the epilogue on full 256x256
    // tiles of bf16 output, where C is then not written; otherwise the product goes to C and
    // swiglu_bwd runs after it.
    const void* dglu_gu = nullptr;
    void* dglu_out = nullptr;
    int64_t dglu_ld = 0;
    // Optional sums of squares of the stored output (fp32 C only), for the gradient norm: the
    // call writes one fp64 partial and one non-finite flag per slot into sq_part[0..) /
    // sq_nf[0..) (at most sq_cap slots; how many depends on the path, always the same for the
    // same shapes) and leaves the rest of the region alone.  Each partial adds double(x0^2 +
    // x1^2) + double(x2^2 + x3^2) over groups of four stored values, as sqnorm_k does.  The
    // tile kernels do it in their epilogue (or split-K reduction); other paths read C back.
    double* sq_part = nullptr;
    int* sq_nf = nullptr;
    int64_t sq_cap = 0;
};

bool gemm_mfma_eligible(const GemmArgs& a);
// The INT4 B operand in the kernel: bf16 A (not transposed, lda % 8, 16-byte aligned), K a
// positive multiple of 64, M and N >= 8, fp16 scales (4-byte aligned base), group % 64 == 0,
// ldb % 64 == 0, Bq 16-byte aligned, N a multiple of 64 for the input-gradient layout, fewer
// than 2^38 weight elements.
bool gemm_q4_eligible(const GemmArgs& a);
bool gemm_dma_eligible(const GemmArgs& a);
void gemm(const GemmArgs& a, hipStream_t stream);
// Independent products in one launch when they share the kernel configuration (transposes,
// dtypes, alpha, beta; no residual or low-rank term; up to 8), so that their tiles fill the
// chip together instead of each product's last partial round; otherwise one gemm() each.
// Sums of squares (sq_*) of the whole call go to a[0]'s slot region; the others' are ignored.
void gemm_grouped(const GemmArgs* a, int n, hipStream_t stream);

// The products of E experts over row-ragged operands, one launch, with the row ranges read on
// the device (no host round trip to size them).  Expert e owns the rows [offsets[e],
// offsets[e+1]) of the row-ragged operands (offsets: E + 1 device int64 values, each a
// multiple of 64, non-decreasing).  `g` describes expert 0's product at row offset 0:
//   ragged M (ragged_k = 0; g.transA = 0): rows of A and C are ragged, g.M is a bound on
//     offsets[E]; expert e uses B + e * b_stride;
//   ragged K (ragged_k = 1; g.transA = 1, g.transB = 0): the K rows of A and B are ragged;
//     expert e writes C + e * c_stride (all zeros when it owns no rows).
// bf16 operands, no residual, no low-rank term; g.K (ragged M) a multiple of 64.
struct RaggedArgs {
    GemmArgs g;
    const int64_t* offsets = nullptr;
    int E = 0;
    int ragged_k = 0;
    int64_t b_stride = 0, c_stride = 0;
};
bool gemm_ragged_eligible(const RaggedArgs& r);
void gemm_ragged(const RaggedArgs& r, hipStream_t stream);

// Upper bounds of the sum-of-squares slots (GemmArgs::sq_*) that a call writes, whichever of its
// paths runs, from the products' M and N only: gemm() (n == 1) or gemm_grouped() (n >= 2) over
// the products a[0..n); gemm_ragged() with ragged K over E experts of an M x N product.  A caller
// that sizes the slot region from these never meets the launchers' "slots needed" checks.
int64_t gemm_sq_slots(const GemmArgs* a, int n);
int64_t gemm_ragged_sq_slots(int64_t M, int64_t N, int E);

}  // namespace aic::hip
