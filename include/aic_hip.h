/*
 * aic_hip.h -- C-ABI of the MI355X (gfx950) backend for the AutonomousAICore TransformerLM
 * training step.
 *
 * Conventions (all entry points):
 *   - return 0 on success, else an aic error code (the numbering of the reference's
 *     aic::ErrorCode, include/core/error.hpp:13-29; 7 = HIP error); no exception crosses
 *     the ABI.  aic_hip_last_error() gives the message of the calling thread's last error.
 *   - pointers are device pointers unless the name says host; sizes are int64_t; row-major
 *     layouts with explicit leading dimensions (in elements).
 *   - the caller allocates outputs (as the reference's raw-pointer launchers do,
 *     e.g. src/ops/flash_attention.cpp:299-300); internal scratch comes from the library's
 *     stream-ordered pool.
 *   - `stream` is a hipStream_t (NULL = the null stream); every call is asynchronous with
 *     respect to the host unless stated.
 * Each declaration names the reference interface it replaces (paths relative to
 * AutonomousAICore/ of the reference repository).
 */
#ifndef AIC_HIP_H
#define AIC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types; values equal the reference's aic::DType (include/core/dtype.hpp:18-26). */
typedef enum {
    AIC_F32 = 0,
    AIC_F16 = 1,
    AIC_BF16 = 2,
    AIC_I32 = 3,
    AIC_I64 = 4,
    AIC_U8 = 5,
    AIC_U16 = 6
} aic_dtype;

typedef void* aic_stream; /* hipStream_t */

/* ---------------------------------------------------------------- runtime ---------- */
/* Message of this thread's last failed call ("" if none).
 * Replaces: aic::Error::what() of AIC_THROW(CudaError, ...) (include/core/error.hpp:31-48). */
const char* aic_hip_last_error(void);
/* Number of visible GPUs (0 without a GPU; never fails).
 * Replaces: get_cuda_device_count (src/runtime/cuda_info.cpp:15-33). */
int aic_hip_device_count(void);
/* Library version string. */
const char* aic_hip_version(void);

/* Stream-ordered caching allocator over hipMallocAsync on the device's default pool, with
 * the release threshold raised so freed blocks stay cached.
 * Replaces: DeviceMemoryPool::allocate_on_stream / deallocate_on_stream
 * (include/memory/memory_pool.hpp:120-155, src/memory/memory_pool.cpp:182-286). */
int aic_hip_mem_alloc_async(void** ptr, size_t bytes, aic_stream stream);
int aic_hip_mem_free_async(void* ptr, aic_stream stream);
/* Bytes currently allocated through the pool and the high-water mark
 * (replaces MemoryStats, include/memory/allocator.hpp:14-50). */
int aic_hip_mem_stats(int64_t* allocated_bytes, int64_t* peak_bytes);
/* Returns the scratch buffers the library keeps cached for `stream` (kernels' partial results,
 * stream-ordered) to the pool.  Call it before destroying a stream the library has run work on:
 * the cache is keyed by the stream handle, so its buffers would otherwise stay allocated, and a
 * later stream created at the same address would inherit them.  The library does this itself
 * for the streams it creates.  No reference counterpart (the reference allocates per call). */
int aic_hip_mem_release_stream(aic_stream stream);
/* Copy of `bytes` between any two of host and device memory, ordered on the stream, returning
 * when it is done (hipMemcpyDefault: the direction comes from the pointers).
 * Replaces: the reference's raw cudaMemcpy calls (e.g. src/tensor/tensor.cpp:266,320,
 * src/cuda/cuda_loss.cu:228-234). */
int aic_hip_memcpy_sync(void* dst, const void* src, size_t bytes, aic_stream stream);

/* ---------------------------------------------------------------- GEMM ------------- */
/* C[M,N] = alpha * op(A) . op(B) + beta * C + R  (fp32 accumulation).
 *   op(A): M x K, stored A[m*lda + k], or A[k*lda + m] when transA.
 *   op(B): K x N, stored B[k*ldb + n], or B[n*ldb + k] when transB.
 *   ab_type: AIC_BF16 (MFMA path) or AIC_F32; c_type: AIC_BF16 or AIC_F32; R (nullable)
 *   has c_type and leading dimension ldr; beta == 0 never reads C.
 * Linear forward y = x W^T is (0, 1); dx = dy W is (0, 0); dW = dy^T x is (1, 0).
 * Replaces: aic::cuda::gemm_2d / matmul (src/cuda/cuda_gemm.cuh:11-14) and the
 * MatMulBackward products (src/autograd/functions.cpp:254-273). */
int aic_hip_gemm(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha, const void* A, int64_t lda,
                 const void* B, int64_t ldb, float beta, void* C, int64_t ldc, const void* R, int64_t ldr,
                 aic_dtype ab_type, aic_dtype c_type, aic_stream stream);

/* The same product with a low-rank term added before scaling (a LoRA projection in one pass):
 *   C = alpha * (op(A) op(B) + X2 Y2^T) + beta * C + R
 * X2 [M, r2] row-major (ldx2); with seg_n > 0 the output columns [s*seg_n, (s+1)*seg_n) take the
 * X2 columns [s*r2, (s+1)*r2) (q, k, v or gate, up stacked in one product); Y2 [N, r2] row-major
 * (ldy2), or [r2, N] when y2_kmajor.  X2 / Y2 have dtype ab_type.  On the bf16 MFMA path the
 * term is accumulated in the product's own registers.
 * Replaces: the sum y = base(x) + lora_B(lora_A(x)) * scaling of LoRALinear::forward
 * (src/nn/lora.cpp:75-93) and the input-gradient sum of its backward. */
int aic_hip_gemm_lowrank(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha, const void* A,
                         int64_t lda, const void* B, int64_t ldb, const void* X2, int64_t ldx2, const void* Y2,
                         int64_t ldy2, int64_t r2, int64_t seg_n, int y2_kmajor, float beta, void* C, int64_t ldc,
                         const void* R, int64_t ldr, aic_dtype ab_type, aic_dtype c_type, aic_stream stream);

/* The attention input projection with the rotary embedding applied on the way out: C = A W^T
 * (bf16 A [M, K], W [N, K], C [M, N]) whose columns [0, rope_cols) are heads of hd values
 * rotated by the half-split RoPE at position start_pos + row % seq (cos_t / sin_t: [positions]
 * [hd / 2] tables as aic_hip_rope_tables builds them).  In the GEMM's epilogue for hd 128 on
 * shapes of at least 128 full 256 x 256 tiles; otherwise the product and then aic_hip_rope.
 * Replaces: Linear (q, k, v projections) followed by RotaryPositionEmbedding::forward on q and
 * k (include/nn/rope.hpp:23-112) as CausalSelfAttention::forward runs them. */
int aic_hip_gemm_rope(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* W, int64_t ldw,
                      void* C, int64_t ldc, int64_t rope_cols, int64_t hd, int64_t seq, int64_t start_pos,
                      const float* cos_t, const float* sin_t, aic_stream stream);

/* The FFN's gate/up projection with SwiGLU applied on the way out: GU = A W^T (bf16 A [M, K],
 * W [2f, K] = the gate rows then the up rows, GU [M, 2f]) and H[row][j] = silu(GU[row][j]) *
 * GU[row][f + j] (bf16 [M, f]).  In the GEMM's epilogue on shapes of at least 128 full 256 x 256
 * tiles with f % 128 == 0; otherwise the product and then aic_hip_swiglu_fwd.
 * Replaces: the gate and up Linear layers followed by silu * mul (SwiGLU::forward,
 * include/nn/swiglu.hpp:21-33). */
int aic_hip_gemm_swiglu(int64_t M, int64_t f, int64_t K, const void* A, int64_t lda, const void* W, int64_t ldw,
                        void* GU, int64_t ldgu, void* H, int64_t ldh, aic_stream stream);

/* The FFN's down-projection input gradient fed straight into SwiGLU's backward: with
 * dh = A B (bf16 A [M, K], B [K, f]; dh [M, f] in DH, leading dimension lddh), g = GU[row][j],
 * u = GU[row][f + j]: DGU[row][j] = dh u silu'(g), DGU[row][f + j] = dh silu(g) (bf16, as
 * aic_hip_swiglu_bwd).  In the GEMM's epilogue on shapes of at least 128 full 256 x 256 tiles,
 * where DH is then not written; otherwise the product goes to DH and aic_hip_swiglu_bwd runs.
 * Replaces: the down Linear layer's input gradient followed by the silu * mul backward
 * (include/nn/swiglu.hpp:21-33, src/autograd/functions.cpp:60-68,167-175). */
int aic_hip_gemm_swiglu_bwd(int64_t M, int64_t f, int64_t K, const void* A, int64_t lda, const void* B, int64_t ldb,
                            const void* GU, int64_t ldgu, void* DH, int64_t lddh, void* DGU, aic_stream stream);

/* LoRA adapter products in one pass over a bf16 operand Y [T, N] (leading dimension ldy) whose
 * columns form N / n_seg segments of n_seg columns (n_seg % 256 == 0), segment g paired with
 * columns [g r_seg, (g+1) r_seg) of the small operands (r_seg 16, 32 or 48):
 *   out1[t, g r_seg + j] = bf16(scale * sum_{n in segment g} Y[t, n] W(n, j))  (out1 non-NULL)
 *   out2(n, j) (+)= sum_t Y[t, n] Z[t, g(n) r_seg + j]                         (out2 non-NULL)
 * W(n, j) = W[n w_n + j w_j] with w_j == 1 (B [out, r] rows) or w_n == 1 (A [r, in] rows);
 * out1 bf16 [T, ldo1]; Z bf16 [T, ldz]; out2 fp32 at out2 + n o2n + j o2j, overwritten or added
 * to (accumulate).  bf16 inputs 16-byte aligned with leading dimensions % 8 == 0, out1 8-byte
 * aligned with ldo1 % 4 == 0.  Deterministic.
 * Other shapes return NotImplemented (the caller runs GEMMs instead).
 * Replaces (no single reference launcher): the rank-r matmuls of LoRALinear::forward and their
 * autograd gradients (src/nn/lora.cpp:75-93; MatMulBackward, src/autograd/functions.cpp:254-273):
 * x A^T (out1 with W = A), dy^T xs and dy B (out2 and out1 in one pass over dy), dxa^T x (out2). */
int aic_hip_lora_skinny(const void* Y, int64_t ldy, int64_t T, int64_t N, int64_t n_seg, int64_t r_seg, const void* W,
                        int64_t w_n, int64_t w_j, void* out1, int64_t ldo1, float scale, const void* Z, int64_t ldz,
                        float* out2, int64_t o2n, int64_t o2j, int accumulate, aic_stream stream);

/* Several independent products in one launch (for example every expert's projection of an MoE
 * layer, or two weight gradients whose tiles together fill the chip once).  They must share
 * transA, transB, the dtypes, alpha and beta, and take the MFMA path (bf16, 16-byte aligned
 * operands, K % 64 == 0, at most 8 products); otherwise each runs as aic_hip_gemm.
 * Replaces: the per-expert matmul loop of MoELayer::forward / backward
 * (src/nn/moe.cpp:205-245), one launch per expert there. */
typedef struct {
    int transA, transB;
    int64_t M, N, K;
    const void* A;
    int64_t lda;
    const void* B;
    int64_t ldb;
    void* C;
    int64_t ldc;
} aic_gemm_desc;
int aic_hip_gemm_grouped(int n, const aic_gemm_desc* descs, float alpha, float beta, aic_dtype ab_type,
                         aic_dtype c_type, aic_stream stream);

/* Expert-ragged product: expert e's rows are [offsets[e], offsets[e+1]) of A and C (offsets: E + 1
 * int64 on the device, read by the kernels -- no host synchronisation), and
 *   C[rows_e] = alpha * A[rows_e] op(B_e),  B_e = B + e * b_stride elements,
 * op(B_e) = B_e^T ([N, K] rows, transB = 1) or B_e ([K, N], transB = 0); bf16 A and B, C bf16 or
 * fp32 [M, ldc] (M: a bound on the rows, the buffers' size).  SwiGLU in the epilogue as
 * aic_hip_gemm_swiglu / aic_hip_gemm_swiglu_bwd: glu_f > 0 (transB = 1, N = 2 glu_f) also writes
 * glu_out[row][j] = silu(C[row][j]) C[row][glu_f + j]; dglu_gu non-NULL (transB = 0) writes
 * dglu_out from the product dh and the saved gate/up rows dglu_gu (C then need not be written).
 * Where the epilogue does not take the shape (N % 256 != 0, or glu_f % 128 != 0), the product goes
 * to C and the standalone SwiGLU pass runs over all M rows.  Shapes the kernels do not take
 * return NotImplemented.
 * Replaces: the per-expert matmul loop of MoELayer::forward / backward (src/nn/moe.cpp:205-245),
 * one launch per expert there, with the host reading the expert counts. */
int aic_hip_gemm_ragged(int transB, int64_t M, int64_t N, int64_t K, float alpha, const void* A, int64_t lda,
                        const void* B, int64_t ldb, int64_t b_stride, void* C, int64_t ldc, const int64_t* offsets,
                        int E, int64_t glu_f, void* glu_out, int64_t ld_glu, const void* dglu_gu, void* dglu_out,
                        int64_t dglu_ld, aic_dtype c_type, aic_stream stream);

/* ---------------------------------------------------------------- RMSNorm ---------- */
/* y = x / rms * w with rms = sqrt(mean(x^2) + eps) per row; rms[rows] (fp32) is saved.
 * x/y have dtype dt (F32 or BF16), leading dimensions ldx/ldy; w is fp32 [dim].
 * Replaces: the RMSNorm composite (include/nn/rms_norm.hpp:18-34). */
int aic_hip_rmsnorm_fwd(const void* x, int64_t ldx, const float* w, void* y, int64_t ldy, float* rms, int64_t rows,
                        int64_t dim, float eps, aic_dtype dt, aic_stream stream);
/* dx = dy*w/rms - x * sum(dy*w*x)/(dim*rms^3) (+ dres if non-NULL, the residual-stream
 * gradient, fused);  dw (fp32 [dim]) = sum_rows dy*x/rms, overwritten (accumulate = 0) or
 * added to (accumulate = 1).  dw may be NULL.  dx may alias dres.
 * Replaces: the backward of the same composite (src/autograd/functions.cpp:60-200). */
int aic_hip_rmsnorm_bwd(const void* dy, int64_t lddy, const void* x, int64_t ldx, const float* w, const float* rms,
                        const void* dres, int64_t ldres, void* dx, int64_t lddx, float* dw, int accumulate, int64_t rows,
                        int64_t dim, aic_dtype dt, aic_stream stream);

/* ---------------------------------------------------------------- RoPE ------------- */
/* In-place half-split rotation of `heads` heads of width hd per row:
 *   row t = b*S + s (position start_pos + s), head h at x[t*ld + h*hd + i].
 * inverse = 0: x1' = x1 c - x2 s, x2' = x1 s + x2 c; inverse = 1: the adjoint (backward).
 * cos_t/sin_t: fp32 [>= start_pos+S, hd/2], as built by aic_hip_rope_tables.
 * q and k of a fused [T, 3d] projection are rotated by one call with heads = 2*n_heads.
 * Replaces: RotaryPositionEmbedding::forward and RoPEBackward (include/nn/rope.hpp:23-112). */
int aic_hip_rope(void* x, int64_t ld, int64_t B, int64_t S, int64_t heads, int64_t hd, int64_t start_pos,
                 const float* cos_t, const float* sin_t, int inverse, aic_dtype dt, aic_stream stream);
/* Host: fill host arrays cos_t/sin_t [max_seq, hd/2] exactly as the reference builds its
 * cache in float (include/nn/rope.hpp:122-144). */
int aic_hip_rope_tables(float* cos_host, float* sin_host, int64_t max_seq, int64_t hd, float base);

/* ---------------------------------------------------------------- attention -------- */
/* Causal flash attention forward.  q/k/v rows are tokens t = b*S + s with head h at
 * column h*hd (leading dimension ld_qkv, e.g. 3*d for a fused QKV projection); o has
 * leading dimension ld_o; lse [B, H, S] fp32 (natural-log row log-sum-exp of the scaled
 * scores).  hd in {32, 64, 128}; dt F32 or BF16.
 * Replaces: launch_flash_attention_forward_gpu (src/cuda/cuda_flash_attention.cuh:12-28)
 * and the default materialised path (include/nn/attention.hpp:84-119). */
int aic_hip_attn_fwd(const void* q, const void* k, const void* v, int64_t ld_qkv, void* o, int64_t ld_o, float* lse,
                     int64_t B, int64_t H, int64_t S, int64_t hd, int causal, float scale, aic_dtype dt,
                     aic_stream stream);
/* Backward: dq/dk/dv (leading dimension ld_d) from o, do (leading dimension ld_o) and lse.
 * Deterministic (no atomics).
 * Replaces: launch_flash_attention_backward_gpu (src/cuda/cuda_flash_attention.cuh:30-46). */
int aic_hip_attn_bwd(const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o, const void* dout,
                     int64_t ld_o, const float* lse, void* dq, void* dk, void* dv, int64_t ld_d, int64_t B, int64_t H,
                     int64_t S, int64_t hd, int causal, float scale, aic_dtype dt, aic_stream stream);
/* The same with the half-split rotary embedding's backward applied to dq and dk on the way out
 * (cos_t / sin_t: [S][hd / 2] tables as aic_hip_rope_tables builds them, positions 0..S-1 of
 * each sequence), as the attention layer's backward runs it right after the attention.
 * Replaces: launch_flash_attention_backward_gpu followed by RoPEBackward on the q and k
 * gradients (src/cuda/cuda_flash_attention.cuh:30-46, include/nn/rope.hpp:23-112). */
int aic_hip_attn_bwd_rope(const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o, const void* dout,
                          int64_t ld_o, const float* lse, void* dq, void* dk, void* dv, int64_t ld_d, int64_t B,
                          int64_t H, int64_t S, int64_t hd, int causal, float scale, const float* cos_t,
                          const float* sin_t, aic_dtype dt, aic_stream stream);

/* Queries and keys of different lengths (seq_len_q != seq_len_k): q, o, do rows are tokens
 * b*Sq + s (leading dimensions ld_q, ld_o), k, v rows b*Sk + s (ld_k); dq has leading dimension
 * ld_dq, dk and dv ld_dkv; lse [B, H, Sq].  Causal as the reference's CPU path: query r sees the
 * keys c <= r.  fp32 math for F32 and BF16 (any Sq, Sk > 0; Sq == Sk is also accepted; with
 * Sq == 0 the backward writes zero dk and dv).  head_dim 16, 32, 64 or 128.
 * Replaces: launch_flash_attention_forward_gpu / launch_flash_attention_backward_gpu with
 * seq_len_q != seq_len_k (src/cuda/cuda_flash_attention.cuh:12-46; src/ops/flash_attention.cpp:
 * 32-260 on the CPU). */
int aic_hip_attn_fwd_qk(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_k, void* o, int64_t ld_o,
                        float* lse, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t hd, int causal, float scale,
                        aic_dtype dt, aic_stream stream);
int aic_hip_attn_bwd_qk(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_k, const void* o,
                        const void* dout, int64_t ld_o, const float* lse, void* dq, int64_t ld_dq, void* dk, void* dv,
                        int64_t ld_dkv, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t hd, int causal,
                        float scale, aic_dtype dt, aic_stream stream);

/* ---------------------------------------------------------------- SwiGLU ----------- */
/* h = silu(g) * u, silu(x) = x / (1 + exp(-x)); g, u, h [T, f] with leading dims ld_gu, ld_h.
 * Replaces: silu + mul of SwiGLU::forward (include/nn/swiglu.hpp:21-33). */
int aic_hip_swiglu_fwd(const void* g, const void* u, int64_t ld_gu, void* h, int64_t ld_h, int64_t T, int64_t f,
                       aic_dtype dt, aic_stream stream);
/* dg = dh*u*silu'(g), du = dh*silu(g), silu'(x) = s(1+x(1-s)).
 * Replaces: SiluBackward + MulBackward (src/autograd/functions.cpp:60-68,167-175). */
int aic_hip_swiglu_bwd(const void* g, const void* u, int64_t ld_gu, const void* dh, int64_t ld_h, void* dg, void* du,
                       int64_t ld_d, int64_t T, int64_t f, aic_dtype dt, aic_stream stream);

/* ---------------------------------------------------------------- cross-entropy ---- */
/* Per-row LSE loss with index targets; losses[N], lse[N] (fp32, may be NULL except lse
 * when a backward follows); *loss_mean (device fp32) = sum(losses)/valid, *valid (device
 * int64) = rows with target != ignore_index.  Deterministic.  A target outside [0, C) other
 * than ignore_index is a valid row with loss lse - 0 (and gradient softmax, no one-hot), as the
 * CUDA launcher computes it (src/cuda/cuda_loss.cu:114-121).
 * Replaces: cuda_cross_entropy_forward (src/cuda/cuda_loss.cuh:17-33). */
int aic_hip_ce_fwd(const void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
                   float* losses, float* lse, float* loss_mean, int64_t* valid, aic_dtype dt, aic_stream stream);
/* dlogits = (exp(z - lse) - onehot(t)) * (*grad) / (*valid); ignored rows are 0.
 * grad and valid are device scalars; dlogits may alias logits.
 * Replaces: cuda_cross_entropy_backward (src/cuda/cuda_loss.cuh:35-52). */
int aic_hip_ce_bwd(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                   int64_t ignore_index, const float* grad, const int64_t* valid, void* dlogits, int64_t ld_d,
                   aic_dtype dt, aic_stream stream);

/* The gradient with the reference launcher's reductions (CrossEntropyBackward,
 * src/loss/cross_entropy.cpp:86-105): dlogits[i,:] = (softmax(z_i) - onehot(t_i)) * w_i,
 * ignored rows 0, where w_i = grad[i] for reduction "none" (per_row = 1; grad NULL: 1), and
 * otherwise w_i = grad[0] / divisor (grad NULL: 1 / divisor; divisor 0: w_i = 0) with divisor =
 * the host's valid-row count for "mean" and 1 for "sum".  grad is a device pointer.
 * Replaces: cuda_cross_entropy_backward (src/cuda/cuda_loss.cuh:35-52) with its reduction
 * string and host valid_count. */
int aic_hip_ce_bwd_rows(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N,
                        int64_t C, int64_t ignore_index, const float* grad, int per_row, float divisor, void* dlogits,
                        int64_t ld_d, aic_dtype dt, aic_stream stream);
/* Forward and backward of the mean loss in one pass over the logits: losses, lse, *loss_mean and
 * *valid as aic_hip_ce_fwd (valid required), and the logits overwritten by the gradient of
 * aic_hip_ce_bwd with grad (device scalar; NULL: 1).  bf16 rows of C % 8 == 0 up to 65536 are
 * read once into registers and written once; other shapes run the two passes.  Results equal
 * aic_hip_ce_fwd followed by aic_hip_ce_bwd bit for bit.
 * Replaces: cuda_cross_entropy_forward + cuda_cross_entropy_backward (src/cuda/cuda_loss.cuh:
 * 17-52) as CrossEntropyLoss::forward and its backward call them for one loss. */
int aic_hip_ce_fwd_bwd(void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
                       float* losses, float* lse, float* loss_mean, int64_t* valid, const float* grad, aic_dtype dt,
                       aic_stream stream);
/* Soft (probability) targets y [N, C] fp32 with leading dimension ld_y: losses[i] = lse_i -
 * sum_j y_ij z_ij, every row valid, *loss_mean = sum(losses) / N (any of losses, lse, loss_mean
 * may be NULL; lse is needed by the backward).  The backward writes dlogits = (softmax(z) - y) * w_i
 * with w_i as aic_hip_ce_bwd_rows (per_row, grad, divisor: N for "mean", 1 for "sum").
 * Replaces: cuda_cross_entropy_forward / cuda_cross_entropy_backward with soft_targets
 * (src/cuda/cuda_loss.cu:123-131, 177-184; src/loss/cross_entropy.cpp:208-260 on the CPU). */
int aic_hip_ce_fwd_soft(const void* logits, int64_t ld, const float* y, int64_t ld_y, int64_t N, int64_t C,
                        float* losses, float* lse, float* loss_mean, aic_dtype dt, aic_stream stream);
int aic_hip_ce_bwd_soft(const void* logits, int64_t ld, const float* y, int64_t ld_y, const float* lse, int64_t N,
                        int64_t C, const float* grad, int per_row, float divisor, void* dlogits, int64_t ld_d,
                        aic_dtype dt, aic_stream stream);

/* ---------------------------------------------------------------- embedding -------- */
/* out[i,:] = W[ids[i],:] (zero row for ids outside [0, V)); W/out dtype dt.
 * Replaces: cuda_embedding_forward (src/cuda/cuda_embedding.cuh:10-18). */
int aic_hip_embed_fwd(const int64_t* ids, int64_t N, const void* W, int64_t V, int64_t D, void* out, aic_dtype dt,
                      aic_stream stream);
/* dW[v,:] (fp32) = sum over i with ids[i] == v of dout[i,:], summed in a fixed order
 * (deterministic; no atomics); overwrite (accumulate = 0: rows of absent ids become 0)
 * or add (accumulate = 1).  N <= 2^20 tokens per call; no memset (safe to capture).
 * Replaces: cuda_embedding_backward (src/cuda/cuda_embedding.cuh:20-28). */
int aic_hip_embed_bwd(const int64_t* ids, int64_t N, const void* dout, int64_t V, int64_t D, float* dW, int accumulate,
                      aic_dtype dt, aic_stream stream);

/* ---------------------------------------------------------------- optimizer -------- */
/* Sum of squares (fp64) of `count` fp32 gradient buffers, and a non-finite flag, written to
 * the device scalars *sqnorm and *nonfinite.  grads/sizes are host arrays of device
 * pointers / element counts.
 * Replaces: the per-parameter mul + sum + .item() of clip_grad_norm_
 * (src/optim/clip_grad.cpp:33-37) and launch_has_nan_or_inf_gpu (src/train/amp.cpp:12-15). */
int aic_hip_grad_sqnorm_multi(const float* const* grads, const int64_t* sizes, int count, double* sqnorm,
                              int* nonfinite, aic_stream stream);
/* aic_hip_grad_sqnorm_multi without any device allocation, for callers that cannot allocate
 * (code under HIP graph capture, tight serving or training loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments and results, bit for bit;
 * the fp64 partials live in a fixed per-device array of the library (1.5 MiB, held until
 * the process ends) instead of allocated scratch.  Limit: the tensors' partial blocks,
 * min(ceil(n / 4096), 1024) per tensor, may total at most 131072 (e.g. 128 tensors of
 * 4 M elements or more); beyond that it returns OutOfRange and launches nothing.  Every call
 * on one device shares the array, so calls that overlap in time on one device (other
 * streams, other threads) race; calls ordered on one stream do not. */
int aic_hip_grad_sqnorm_multi_noalloc(const float* const* grads, const int64_t* sizes, int count, double* sqnorm,
                                      int* nonfinite, aic_stream stream);
/* grads[i] *= (*scale) for every buffer (device scalar).
 * Replaces: launch_unscale_gpu (src/train/amp.cpp:12-15) and mul_ of clip_grad_norm_
 * (src/optim/clip_grad.cpp:45-50). */
int aic_hip_scale_multi(float* const* grads, const int64_t* sizes, int count, const float* scale, aic_stream stream);

/* Device-resident optimizer control block: loss scaler state (src/train/amp.cpp:50-152)
 * and the outputs of the clip decision.  Lives in device memory. */
typedef struct {
    float scale;           /* current loss scale (1 when scaling is off) */
    int good_steps;
    int skipped_steps;
    int use_scaler;
    float growth_factor, backoff_factor;
    int growth_interval;
    float min_scale, max_scale;
    float max_grad_norm;   /* <= 0: no clipping */
    float grad_norm;       /* out: pre-clip L2 norm of the unscaled gradients */
    float grad_mult;       /* out: multiplier AdamW applies to the raw gradient (clip/scale) */
    int skip;              /* out: 1 when a non-finite gradient was found (step skipped) */
    int step;              /* AdamW step count; finalize increments it when the step is applied */
} aic_optim_ctl;

/* One thread: from *sqnorm and *nonfinite decide skip / backoff / growth exactly as
 * DynamicLossScaler::unscale_and_update, then norm = sqrt(sqnorm)/scale and the clip
 * coefficient max/(norm + 1e-6) when < 1 (clip_grad_norm_), leaving grad_mult =
 * coef/scale for AdamW, and increments step unless the step is skipped.  The scale used
 * for this step is the one on entry.
 * Replaces: the host logic of src/train/amp.cpp:118-152 and src/optim/clip_grad.cpp:40-50. */
int aic_hip_optim_finalize(const double* sqnorm, const int* nonfinite, aic_optim_ctl* ctl, aic_stream stream);

/* Fused AdamW over `count` tensors (host arrays of device pointers / sizes):
 *   g' = g * ctl->grad_mult (or g when ctl is NULL); skip everything when ctl->skip;
 *   the step count is ctl->step when ctl is non-NULL, else `step`;
 *   p -= lr*wd*p; m = b1 m + (1-b1) g'; v = b2 v + (1-b2) g'^2;
 *   p -= lr * (m/bc1) / (sqrt(v/bc2) + eps), bc_i = 1 - beta_i^step (float).
 * p_bf16[i] (nullable entries) receive the bf16 copy of the updated parameter.
 * Replaces: cuda_adamw_step (src/cuda/cuda_adamw.cuh:10-24), one launch for all tensors. */
int aic_hip_adamw_multi(float* const* p, const float* const* g, float* const* m, float* const* v, void* const* p_bf16,
                        const int64_t* sizes, int count, float lr, float beta1, float beta2, float eps,
                        float weight_decay, int64_t step, const aic_optim_ctl* ctl, aic_stream stream);

/* AdamW on one tensor with the caller's bias corrections bc1 = 1 - beta1^t and
 * bc2 = 1 - beta2^t (computed in float on the host, as AdamW::step does,
 * src/optim/adamw.cpp:28-29); same update order as aic_hip_adamw_multi.
 * Replaces: cuda_adamw_step (src/cuda/cuda_adamw.cuh:10-24), argument for argument. */
int aic_hip_adamw_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                       float eps, float weight_decay, float bias_correction1, float bias_correction2,
                       aic_stream stream);

/* fp32 -> bf16 (round to nearest even) copy of n elements. */
int aic_hip_cast_f32_bf16(const float* src, void* dst, int64_t n, aic_stream stream);

/* Streaming probe over n fp32 elements (n a multiple of 4; fp32 buffers 16-byte aligned):
 *   out[j][i] = sum_k in[k][i] + j  (j < n_out),  out_bf16[i] = bf16(sum_k in[k][i])  (nullable);
 * with no output at all, sink[0] may receive 0.  One pass in the form of the AdamW kernel (two
 * float4 groups per thread, grid-stride), plain or non-temporal accesses.  Mixes: (n_in, n_out,
 * bf16) = (1,0,no) read, (0,1,no) write, (1,1,no) copy, (2,1,no) add, (4,3,yes) AdamW's bytes.
 * No counterpart in the reference: it measures the HBM rate the bandwidth-bound kernels are
 * judged against. */
int aic_hip_stream_probe(const float* const* in, int n_in, float* const* out, int n_out, void* out_bf16, float* sink,
                         int64_t n, int nontemporal, aic_stream stream);

/* ---------------------------------------------------------------- mixture of experts */
/* Routing on fp32 gate logits [T,E] (E <= 64, top_k <= min(E, 8)): probs = softmax(logits)
 * [T,E]; idx [T,k] = the k largest logits per token, descending, ties to the lower expert
 * index; gsel [T,k] = probs of the selected experts divided by their sum + 1e-9 (the
 * normalised gates of MoELayer::forward); rweights [T,k] (nullable) = softmax over the
 * selected logits (route()'s routing_weights); counts [E] (int64); mean_probs [E] (nullable);
 * *aux = sum_e mean_probs[e] * counts[e] * E * coef / (T * k) (0 when coef <= 0 or E == 1).
 * All outputs in device memory; deterministic (no atomics).
 * Replaces: MoERouter::route (src/nn/moe.cpp:33-129) and the gate normalisation of
 * MoELayer::forward (src/nn/moe.cpp:170-204). */
int aic_hip_moe_route(const float* logits, int64_t T, int64_t E, int64_t k, float aux_coef, int64_t* idx, float* gsel,
                      float* probs, float* rweights, int64_t* counts, float* mean_probs, float* aux, aic_stream stream);
/* Rows needed by the expert-sorted layout: T*k entries plus padding to 64-row expert blocks. */
int64_t aic_hip_moe_max_rows(int64_t T, int64_t E, int64_t k);
/* Stable dispatch order: expert e owns rows [offsets[e], offsets[e+1]) (offsets [E+1], int64,
 * multiples of 64); dst_row [T*k] = row of entry t*k+j; src_ent [max_rows] = entry of a row,
 * -1 for padding.  Tokens keep their order inside an expert.
 * Replaces: the host-side mask and per-expert dense dispatch of MoELayer::forward
 * (src/nn/moe.cpp:177-246). */
int aic_hip_moe_permute(const int64_t* idx, const int64_t* counts, int64_t T, int64_t k, int64_t E, int64_t* offsets,
                        int32_t* dst_row, int32_t* src_ent, aic_stream stream);
/* xp[r,:] = x[token of src_ent[r],:] (zero rows for padding). */
int aic_hip_moe_gather(const void* x, int64_t ldx, const int32_t* src_ent, int64_t k, int64_t rows, int64_t d,
                       void* xp, aic_dtype dt, aic_stream stream);
/* Un-permute: out[t,:] = residual[t,:] (nullable) + sum over the token's experts, in increasing
 * expert index, of gsel[t,j] * ye[dst_row[t*k+j],:].
 * Replaces: the gate-weighted accumulation of MoELayer::forward (src/nn/moe.cpp:214-246). */
int aic_hip_moe_combine(const void* ye, const int64_t* idx, const int32_t* dst_row, const float* gsel, int64_t T,
                        int64_t k, int64_t d, const void* residual, int64_t ldr, void* out, int64_t ldo, aic_dtype dt,
                        aic_stream stream);

/* The whole MoE feed-forward block (router Linear(d, E), top-k routing with normalised gates
 * and aux loss, E SwiGLU experts on their own tokens, gate-weighted combine) and its backward.
 * Weights: router [E, d]; experts = E consecutive blocks of gate [f,d], up [f,d], down [d,f];
 * all in dt.  Forward: y [T,d] = residual + MoE(h) (residual nullable), *aux (device fp32).
 * The forward keeps h and the weights referenced for the backward.  Backward: dh [T,d] (dt)
 * overwritten; drouter [E,d] and dexperts (fp32, experts layout) overwritten, zero for an
 * expert with no token.
 * Replaces: MoELayer::forward and its autograd graph (src/nn/moe.cpp:155-253). */
typedef struct aic_moe_ffn aic_moe_ffn;
int aic_moe_ffn_create(int64_t d_model, int64_t d_hidden, int64_t num_experts, int64_t top_k, float aux_loss_coef,
                       aic_dtype dt, aic_moe_ffn** out);
int aic_moe_ffn_destroy(aic_moe_ffn* m);
int aic_moe_ffn_forward(aic_moe_ffn* m, const void* h, int64_t T, const void* router_w, const void* experts,
                        const void* residual, void* y, float* aux, aic_stream stream);
int aic_moe_ffn_backward(aic_moe_ffn* m, const void* dy, float daux, void* dh, float* drouter_w, float* dexperts,
                         aic_stream stream);
/* Routing of the last forward, copied to the host: idx [T,k], counts [E] (synchronous). */
int aic_moe_ffn_routing(aic_moe_ffn* m, int64_t* idx_host, int64_t* counts_host, aic_stream stream);

/* ---------------------------------------------------------------- INT4 + LoRA ------ */
/* INT4-symmetric weights: groups of `group` consecutive elements of the flat row-major weight
 * (group <= 0 or > n: one group; an odd group with more than one group is rejected);
 * s = max(absmax/7, 1e-8); q = clamp(round_half_away(x/s), -7, 7); packed[(n+1)/2] holds element
 * 2i in the low nibble and 2i+1 in the high nibble (4-bit two's complement); scales[ceil(n/group)]
 * are AIC_F32 or AIC_F16 (fp16 rounding of the fp32 s, which q always uses).
 * Replaces: QuantizedTensor::quantize, INT4_SYMMETRIC (src/nn/quantization.cpp:197-295), which
 * runs on the host. */
int aic_hip_int4_quantize(const float* x, int64_t n, int64_t group, uint8_t* packed, void* scales,
                          aic_dtype scale_type, aic_stream stream);
/* out[i] = q_i * s_{i/group}, written as out_type (AIC_F32 or AIC_BF16, round to nearest even).
 * Replaces: QuantizedTensor::dequantize (src/nn/quantization.cpp:359-474) and
 * launch_dequantize_int4 (src/cuda/cuda_quantize.cuh; src/cuda/cuda_quantize.cu:141-159). */
int aic_hip_int4_dequantize(const uint8_t* packed, const void* scales, aic_dtype scale_type, int64_t n, int64_t group,
                            void* out, aic_dtype out_type, aic_stream stream);
/* The general INT4 dequantization of the CUDA launcher, argument for argument: element i is the
 * low (even i) or high (odd i) nibble u of packed[i/2], read as 4-bit two's complement when
 * is_signed (u - 16 for u >= 8) or as 0..15 otherwise; g = i / group (group <= 0: 0);
 * out[i] = (val - zero_points[g]) * scales[g] in fp32 (zero_points NULL: 0).  Any group size,
 * odd ones included.  fp32 scales, zero points and output.
 * Replaces: launch_dequantize_int4 (src/cuda/cuda_quantize.cuh; src/cuda/cuda_quantize.cu:54-94,
 * 141-159) for INT4_ASYMMETRIC and unsigned data (src/nn/quantization.cpp:374-379). */
int aic_hip_int4_dequantize_zp(const uint8_t* packed, const float* scales, const float* zero_points, int is_signed,
                               int64_t n, int64_t group, float* out, aic_stream stream);
/* C[M,N] = alpha * X[M,K] . op(deq(Wq)) + beta * C + R with Wq an INT4 weight as above:
 * transW = 1: Wq holds W [N,K] and op(W) = W^T (forward y = x W^T); transW = 0: Wq holds W [K,N]
 * (input gradient dx = dy W).  With bf16 operands (ab_type AIC_BF16) in the shapes the GEMM
 * kernel takes (K % 64 == 0, group % 64 == 0, the weight's row length % 64 == 0, and for
 * transW = 0 N % 64 == 0; M, N >= 8; X and Wq 16-byte aligned) the packed values and scales are
 * read by the GEMM itself and dequantized in its operand load, with no dequantized copy in HBM.
 * Otherwise (and for AIC_F32) the weight is first dequantized into library scratch in ab_type.
 * Either way op(W) holds q * scale rounded to ab_type, so both routes give the same product;
 * X, C and R as in aic_hip_gemm.
 * Replaces: QuantizedLinear::forward (src/nn/quantization.cpp:669-679: dequantize, transpose,
 * matmul) and its MatMulBackward input gradient (src/autograd/functions.cpp:254-273). */
int aic_hip_int4_dequant_gemm(int transW, int64_t M, int64_t N, int64_t K, float alpha, const void* X, int64_t ldx,
                              const uint8_t* Wq, const void* scales, aic_dtype scale_type, int64_t group, float beta,
                              void* C, int64_t ldc, const void* R, int64_t ldr, aic_dtype ab_type, aic_dtype c_type,
                              aic_stream stream);
/* The QLoRA attention input projection with the rotary embedding applied on the way out:
 *   C = X . deq(Wq)^T + X2 . Y2^T
 * (bf16 X [M, K], INT4 Wq holding W [N, K] with fp16 scales per `group` elements, bf16 C [M, N])
 * whose columns [0, rope_cols) are heads of hd values rotated as in aic_hip_gemm_rope.  The
 * low-rank term is optional (r2 0): X2 [M, *] (ldx2) and Y2 [N, r2] (ldy2) bf16, with seg_n > 0
 * giving output columns [s seg_n, (s+1) seg_n) the X2 columns [s r2, (s+1) r2) (the q, k and v
 * adapters side by side).  The rotation follows the whole sum.  In the INT4 GEMM's epilogue for
 * hd 128 on shapes of at least 128 full 256 x 256 tiles whose low-rank term the kernel takes
 * (r2, ldx2 and ldy2 multiples of 8, X2 and Y2 16-byte aligned, seg_n a multiple of 256);
 * otherwise the product and then aic_hip_rope.
 * Replaces: the q, k, v LoRALinear::forward over QuantizedLinear::forward (src/nn/lora.cpp:75-93,
 * src/nn/quantization.cpp:669-679) followed by RotaryPositionEmbedding::forward on q and k
 * (include/nn/rope.hpp:23-112). */
int aic_hip_int4_gemm_rope(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, const uint8_t* Wq,
                           const void* scales, int64_t group, const void* X2, int64_t ldx2, const void* Y2, int64_t ldy2,
                           int64_t r2, int64_t seg_n, void* C, int64_t ldc, int64_t rope_cols, int64_t hd, int64_t seq,
                           int64_t start_pos, const float* cos_t, const float* sin_t, aic_stream stream);
/* The QLoRA FFN's gate/up projection with SwiGLU on the way out: GU = X . deq(Wq)^T + X2 . Y2^T
 * (bf16 X [M, K], INT4 Wq holding W [2f, K] -- gate rows then up rows -- with fp16 scales per
 * `group` elements; GU [M, 2f] bf16) and H[row][j] = silu(GU[row][j]) GU[row][f + j] (bf16 [M, f]),
 * as aic_hip_gemm_swiglu.  The low-rank term is optional (r2 0); seg_n > 0 gives the gate and up
 * columns their own X2 columns (the two adapters side by side, seg_n = f).  In the INT4 GEMM's
 * epilogue on shapes of at least 128 full 256 x 256 tiles with f % 128 == 0 whose weight the
 * operand load takes (K, group and the row length multiples of 64) and whose low-rank term the
 * kernel takes (seg_n a multiple of 256); other shapes return NotImplemented.
 * Replaces: the gate and up LoRALinear::forward over QuantizedLinear::forward (src/nn/lora.cpp:
 * 75-93, src/nn/quantization.cpp:669-679) followed by silu * mul (include/nn/swiglu.hpp:21-33). */
int aic_hip_int4_gemm_swiglu(int64_t M, int64_t f, int64_t K, const void* X, int64_t ldx, const uint8_t* Wq,
                             const void* scales, int64_t group, const void* X2, int64_t ldx2, const void* Y2,
                             int64_t ldy2, int64_t r2, int64_t seg_n, void* GU, int64_t ldgu, void* H, int64_t ldh,
                             aic_stream stream);
/* W[out,in] += sign * scaling * B[out,rank] . A[rank,in]  (sign >= 0: merge, < 0: unmerge);
 * W, A, B of `dtype` (AIC_F32 or AIC_BF16).
 * Replaces: LoRALinear::merge / unmerge (src/nn/lora.cpp:95-108). */
int aic_hip_lora_merge(void* W, const void* A, const void* B, int64_t in_features, int64_t out_features, int64_t rank,
                       float scaling, int sign, aic_dtype dtype, aic_stream stream);

/* A QLoRA projection: frozen INT4 base plus LoRA adapter,
 *   y = x . deq(Wq)^T + ((x . A^T) . B^T) * (alpha / rank)  [+ R],
 * with A [rank,in], B [out,rank]; rank 0 is the plain QuantizedLinear.  dtype (AIC_F32 or
 * AIC_BF16) is the type of x, y, R, dx, A and B; adapter gradients are fp32.
 * Replaces: LoRALinear::forward (src/nn/lora.cpp:75-93) over QuantizedLinear::forward
 * (src/nn/quantization.cpp:669-679), with the base frozen as LoRALinear does (lora.cpp:54-56). */
typedef struct aic_qlora_linear aic_qlora_linear;
int aic_qlora_linear_create(int64_t in_features, int64_t out_features, int64_t rank, float alpha, int64_t group,
                            aic_dtype scale_type, aic_dtype dtype, aic_qlora_linear** out);
int aic_qlora_linear_destroy(aic_qlora_linear* m);
/* x [T,in], y / R [T,out] (R nullable).  x, Wq, scales, A and B stay referenced until backward. */
int aic_qlora_linear_forward(aic_qlora_linear* m, const void* x, int64_t T, const uint8_t* Wq, const void* scales,
                             const void* A, const void* B, const void* R, void* y, aic_stream stream);
/* dy [T,out] -> dx [T,in] (overwritten; NULL skips it), dA [rank,in] and dB [out,rank] (fp32,
 * overwritten, or added to when accumulate != 0, as AccumulateGrad adds). */
int aic_qlora_linear_backward(aic_qlora_linear* m, const void* dy, void* dx, float* dA, float* dB, int accumulate,
                              aic_stream stream);

/* ---------------------------------------------------------------- tensor primitives */
/* fp32 primitives of the reference's tensor backend.  A view is (offset, ndim <= 8, shape,
 * strides), all in elements, with shape/strides host arrays; outputs are contiguous. */
/* Contiguous copy of a strided view (elem_size 1, 2, 4 or 8 bytes).
 * Replaces: Tensor::clone / contiguous (src/tensor/tensor.cpp:248-304), whose GPU path goes
 * through the host. */
int aic_hip_strided_copy(const void* src, int64_t offset, int ndim, const int64_t* shape, const int64_t* strides,
                         int64_t elem_size, void* dst, aic_stream stream);
/* n elements from -> to for the reference's cast table (f32<->f16, f32<->bf16, f32<->i64,
 * f32<->i32, i64<->i32), with its rounding and NaN encodings (include/core/dtype.hpp:65-133);
 * any other pair fails with NotImplemented (8).
 * Replaces: Tensor::to(DType) (src/tensor/tensor.cpp:359-410), a host round trip on the GPU. */
int aic_hip_cast(const void* src, aic_dtype from, void* dst, aic_dtype to, int64_t n, aic_stream stream);
/* out = a (op) b with NumPy broadcasting (op 0 add, 1 sub, 2 mul, 3 div); out has the
 * broadcast shape.  Incompatible shapes fail with ShapeMismatch (3).
 * Replaces: aic::cuda::add/sub/mul/div (src/cuda/cuda_elementwise.cuh:9-12; semantics of
 * src/ops/cpu_ops.cpp:14-101 and src/core/shape.cpp:138-195). */
int aic_hip_binary(int op, const float* a, int64_t a_offset, int a_ndim, const int64_t* a_shape,
                   const int64_t* a_strides, const float* b, int64_t b_offset, int b_ndim, const int64_t* b_shape,
                   const int64_t* b_strides, float* out, aic_stream stream);
/* y = f(x) over n contiguous elements: 0 neg, 1 abs, 2 exp, 3 log, 4 sqrt, 5 tanh, 6 sigmoid,
 * 7 gelu (tanh form), 8 silu.
 * Replaces: aic::cuda::neg ... silu (src/cuda/cuda_elementwise.cuh:14-22; src/ops/cpu_ops.cpp:105-146). */
int aic_hip_unary(int op, const float* x, float* y, int64_t n, aic_stream stream);
/* *out = sum / mean / max / min (op 0..3) of n contiguous elements; sums in double.
 * Replaces: aic::cuda::sum/mean/max/min(a) (src/cuda/cuda_reductions.cuh:10-14; src/ops/cpu_ops.cpp:151-197). */
int aic_hip_reduce_all(int op, const float* x, int64_t n, float* out, aic_stream stream);
/* Reduction of a contiguous tensor along dim (negative counts from the end); out holds the
 * shape without dim (keepdim only changes the shape).
 * Replaces: aic::cuda::sum/mean/max/min(a, dim, keepdim) (src/cuda/cuda_reductions.cuh:15-18;
 * src/ops/cpu_ops.cpp:203-287). */
int aic_hip_reduce_dim(int op, const float* x, int ndim, const int64_t* shape, int dim, float* out, aic_stream stream);
/* Concatenation of count contiguous [outer, mids[i], inner] tensors (device pointers in a host
 * array) into [outer, sum(mids), inner].  Replaces: cat (src/ops/ops.cpp:473-530). */
int aic_hip_cat(const void* const* srcs, const int64_t* mids, int count, int64_t outer, int64_t inner,
                int64_t elem_size, void* dst, aic_stream stream);
/* Sums a broadcast gradient back to target_shape: leading dims, then dims where the target is 1,
 * one float-rounded sum per dim as the reference does.
 * Replaces: reduce_gradient_for_broadcast (src/autograd/functions.cpp:10-41). */
int aic_hip_sum_to_shape(const float* grad, int ndim, const int64_t* shape, int target_ndim,
                         const int64_t* target_shape, float* out, aic_stream stream);

/* ---------------------------------------------------------------- TransformerLM ---- */
/* The whole training step behind the reference's C++ API (TransformerLM::forward,
 * cross_entropy, Tensor::backward, DynamicLossScaler, clip_grad_norm_, AdamW::step;
 * src/train/trainer.cpp:37-118), with parameters, gradients and AdamW state in flat
 * device arenas. */
typedef struct aic_lm aic_lm;

typedef struct {
    int64_t vocab, d_model, n_layers, n_heads, d_ffn, max_seq_len;
    float norm_eps, rope_base;
    int tied;              /* lm_head shares tok_embeddings.weight */
    aic_dtype compute;     /* AIC_F32 (reference precision) or AIC_BF16 (AMP: bf16 compute,
                              fp32 master weights, gradients and AdamW state) */
    int64_t n_experts;     /* 0: dense SwiGLU FFN; > 0: MoETransformerLM (src/models/moe_transformer_lm.cpp):
                              every FFN is n_experts SwiGLU experts of d_ffn with a top_k router,
                              and the loss is cross_entropy + total_aux_loss (<= 64 experts) */
    int64_t top_k;
    float aux_loss_coef;
    int64_t lora_rank;     /* 0: full fine-tuning; > 0: QLoRA (LoRAAdapter::apply over
                              QuantizedLinear::from_linear, src/nn/lora.cpp:116-175,
                              src/nn/quantization.cpp:669-679): the base model is frozen, the seven
                              projections of each layer are INT4-symmetric groups of quant_group
                              elements with fp16 scales, and only rank-lora_rank adapters
                              (scaling lora_alpha / lora_rank) on all seven are trained */
    float lora_alpha;
    int64_t quant_group;
} aic_lm_config;

typedef struct {
    float lr, beta1, beta2, eps, weight_decay;
    float max_grad_norm;   /* <= 0: no clipping */
    int use_loss_scaler;
    float init_scale, growth_factor, backoff_factor;
    int growth_interval;
    float min_scale, max_scale;
} aic_train_config;

typedef struct {
    float loss;
    float grad_norm;
    int found_inf;
    float loss_scale;      /* scale used by this step */
    int64_t step;          /* AdamW step count after this step */
    float aux_loss;        /* MoE: total_aux_loss, included in loss (0 for a dense model) */
} aic_step_stats;

/* One training step's statistics as the device records them after the step (the step
 * history ring holds the last 1024 steps). */
typedef struct {
    int64_t step;          /* AdamW step count after the step */
    float loss;
    float aux_loss;
    float grad_norm;
    float loss_scale;      /* scale used by the step */
    int32_t found_inf;
    int32_t pad;
} aic_step_record;

/* Creates the model on the current device; parameters are zero until set or initialised. */
int aic_lm_create(const aic_lm_config* cfg, const aic_train_config* tcfg, aic_lm** out);
int aic_lm_destroy(aic_lm* lm);
int64_t aic_lm_num_params(const aic_lm* lm);
int aic_lm_num_tensors(const aic_lm* lm);
/* Name (the reference's parameter name), shape and flat offset of parameter tensor i, in
 * arena order (layer-major; name buffer of name_cap bytes, dims of 2 entries). */
int aic_lm_tensor_info(const aic_lm* lm, int i, char* name, int name_cap, int* rank, int64_t* dims, int64_t* offset);
/* QLoRA: the frozen base model's tensors (the dense model's names, shapes and packed order; with
 * lora_rank == 0 the same list as aic_lm_tensor_info), and setting them, after which the seven
 * projections of every layer are quantized again; and reading them back (fp32, packed).
 * InvalidState without QLoRA.
 * Replaces: loading the base weights before LoRAAdapter::apply (src/nn/lora.cpp:116-175). */
int64_t aic_lm_num_base_params(const aic_lm* lm);
int aic_lm_num_base_tensors(const aic_lm* lm);
int aic_lm_base_tensor_info(const aic_lm* lm, int i, char* name, int name_cap, int* rank, int64_t* dims,
                            int64_t* offset);
int aic_lm_set_base_params(aic_lm* lm, const float* host);
int aic_lm_get_base_params(const aic_lm* lm, float* host);
/* Host <-> device copies of the flat fp32 arenas (synchronous); with QLoRA the trainable
 * arena holds the LoRA adapters only. */
int aic_lm_set_params(aic_lm* lm, const float* host);
int aic_lm_get_params(const aic_lm* lm, float* host);
int aic_lm_get_grads(const aic_lm* lm, float* host);
/* MoE models: the top-k expert selection [T, top_k] (int64, each token's experts by falling
 * logit, lower index on ties) that layer `layer` used in the last forward, copied to idx_host
 * (capacity values; synchronises); *tokens receives T.  No counterpart in the reference: its
 * MoERouter::route result is internal (src/nn/moe.cpp:33-129); exposed so that the step can be
 * checked against the CPU path on the same routing. */
int aic_lm_moe_routing(const aic_lm* lm, int64_t layer, int64_t* idx_host, int64_t capacity, int64_t* tokens);
int aic_lm_get_adam_state(const aic_lm* lm, float* m_host, float* v_host, int64_t* step);
/* Synthetic initialisation on the device: N(0, std) for weight matrices and embeddings,
 * ones for norms; residual projections (out_proj, down_proj) times 1/sqrt(2 L) when
 * residual_scaling.  Counter-based (splitmix64 + Box-Muller), seed-determined. */
int aic_lm_init_normal(aic_lm* lm, uint64_t seed, float std, int residual_scaling);
/* One training step on token ids / targets ([B, S] int64, device pointers when
 * on_device, else host).  stats (host, nullable): when non-NULL the call synchronises and
 * fills it; otherwise the step stays asynchronous on the model's stream.
 * Replaces: Trainer::step (src/train/trainer.cpp:37-118) with a fixed learning rate. */
int aic_lm_train_step(aic_lm* lm, const int64_t* ids, const int64_t* targets, int64_t B, int64_t S, int on_device,
                      aic_step_stats* stats);
/* Loss only (no gradient, no update); synchronous. */
int aic_lm_eval_loss(aic_lm* lm, const int64_t* ids, const int64_t* targets, int64_t B, int64_t S, int on_device,
                     float* loss);
/* KV-cached inference.  forward_step: tokens ids [B, S] (device when on_device, else host) at
 * positions start_pos .. start_pos + S - 1 go through the model, their keys and values join
 * the per-layer cache, and their fp32 logits [B * S, V] are written to logits (device memory
 * when on_device, else host; synchronous when host).  start_pos == 0 starts new sequences; a
 * continuation keeps B.  generate: the reference's sampling loop for one sequence (greedy
 * when temperature <= 0.001 or top_k == 1, else temperature / top-k / top-p and
 * std::mt19937_64(seed)); out_tokens (host, capacity n_prompt + max_new_tokens, at least 1)
 * receives the prompt (or {0} when it is empty) followed by the new tokens, *n_out their count;
 * generation stops after eos_token_id when it is >= 0.
 * Replaces: TransformerLM::forward_step and TransformerLM::generate
 * (src/models/transformer_lm.cpp:64-233) with CausalSelfAttention::forward_with_cache
 * (include/nn/attention.hpp:49-120). */
int aic_lm_forward_step(aic_lm* lm, const int64_t* ids, int64_t B, int64_t S, int64_t start_pos, int on_device,
                        float* logits);
int aic_lm_generate(aic_lm* lm, const int64_t* prompt, int64_t n_prompt, int64_t max_new_tokens, float temperature,
                    int top_k, float top_p, int64_t eos_token_id, uint64_t seed, int64_t* out_tokens, int64_t* n_out);
/* generate's sampling step on its own (host only, no GPU): n_draws tokens drawn one after
 * another from the same fp32 logits [V] with one std::mt19937_64(seed), by the rules above.
 * Replaces: the sampling block of TransformerLM::generate (src/models/transformer_lm.cpp:113-213). */
int aic_sample_tokens(const float* logits, int64_t V, float temperature, int top_k, float top_p, uint64_t seed,
                      int64_t n_draws, int64_t* out);
/* Telemetry hooks.  aic_lm_step_history copies (synchronising once) the records of the steps
 * run since the previous call, oldest first, up to cap (*n = count; *dropped = older records
 * the ring overwrote, nullable) -- so a training loop can feed a telemetry tracker without a
 * host synchronisation per step.  aic_lm_snapshot keeps a device-memory copy of the
 * trainable parameters, the AdamW moments and the optimiser / loss-scaler state;
 * aic_lm_restore puts it back (a rollback in HBM, without a checkpoint file).
 * No counterpart in the reference's step (its controller reloads checkpoint files,
 * src/autonomous/controller.cpp:68-236). */
int aic_lm_step_history(aic_lm* lm, aic_step_record* out, int cap, int* n, int64_t* dropped);
int aic_lm_snapshot(aic_lm* lm);
int aic_lm_restore(aic_lm* lm);
/* The model's HIP stream and a full synchronisation of it. */
int aic_lm_stream(const aic_lm* lm, aic_stream* stream);
int aic_lm_synchronize(aic_lm* lm);
/* Statistics of the last step (synchronises). */
int aic_lm_last_stats(aic_lm* lm, aic_step_stats* stats);

/* Per-kernel-class timing of the steps run while profiling is enabled: a pair of HIP events
 * brackets every launch on the model's stream, and each class accumulates its algorithmic
 * FLOPs (MFMA-bound classes) or HBM bytes (bandwidth-bound classes).  Enabling resets the
 * accumulators.  No counterpart in the reference (it times only whole steps with
 * std::chrono, src/train/trainer.cpp:39,100-102). */
typedef struct {
    char name[32];
    int64_t launches;
    double total_ms;
    double flops;          /* algorithmic FLOPs summed over launches */
    double bytes;          /* algorithmic HBM bytes summed over launches */
    int mfma_bound;        /* 1: judge against the bf16 MFMA peak, 0: against HBM bandwidth */
} aic_kernel_stat;
int aic_lm_profile(aic_lm* lm, int enable);
/* Profiling restricted to some classes (bit c = class c, as numbered by
 * aic_lm_profile_class_index; 0 disables): each timed launch adds an event pair to the queue,
 * so a step measurement times only the class it reports. */
int aic_lm_profile_classes(aic_lm* lm, uint32_t class_mask);
int aic_lm_profile_class_index(const char* name);
/* Synchronises, then writes up to cap classes with at least one launch; *n = count. */
int aic_lm_profile_stats(aic_lm* lm, aic_kernel_stat* out, int cap, int* n);

/* Whether the training step forms the gradient norm (clip_grad_norm_ and the loss scaler's
 * non-finite test) from partial sums written by the gradients' producers -- the weight-gradient
 * GEMMs' epilogues, the split-K reductions, then the embedding and norm weights -- instead of a
 * separate pass over every gradient.  On by default where the model allows it (an untied LM
 * head, dense or MoE FFNs; not QLoRA); enable = 0 selects the pass.  *used (may be null) = whether it is now used.
 * The norm is the same sum in another order (fp64 partials of fp32 squares).
 * Replaces: the norm pass of clip_grad_norm_ (src/optim/clip_grad.cpp:11-53). */
int aic_lm_fused_grad_norm(aic_lm* lm, int enable, int* used);

/* ---------------------------------------------------------------- checkpoints ------- */
/* The reference's .aic format (save_checkpoint / load_checkpoint, src/train/checkpoint.cpp:30-186;
 * docs/architecture.md:96-117): header (magic 'AIC0', version 1, step, epoch, best_val_loss,
 * description), then per tensor name, rank, i64 dims, i32 dtype (reference DType numbering),
 * u64 nbytes, data and its Adler-32.  Host memory only; no GPU is needed.
 * aic_checkpoint_write: tensor i has ranks[i] dims, taken in turn from `dims`.
 * aic_checkpoint_verify: reads the whole file, checking magic, version and every checksum
 * (FormatError otherwise); any output may be NULL.
 * aic_checkpoint_module_order: the order in which Module::named_parameters()
 * (include/nn/module.hpp:63-76) visits the given parameter names, as indices into names. */
int aic_checkpoint_write(const char* path, int64_t step, int64_t epoch, float best_val_loss, const char* description,
                         int64_t n, const char* const* names, const int32_t* ranks, const int64_t* dims,
                         const int32_t* dtypes, const void* const* data, const uint64_t* nbytes);
int aic_checkpoint_verify(const char* path, int64_t* num_tensors, int64_t* step, int64_t* epoch, float* best_val_loss);
int aic_checkpoint_module_order(int64_t n, const char* const* names, int64_t* order);
/* Save / load a model.  The parameters (QLoRA: the frozen base and the adapters) are written
 * as fp32 in named_parameters() order, so a file without optimizer state is what the
 * reference's save_checkpoint writes for the same weights.  with_optimizer appends the AdamW
 * moments ("optimizer.exp_avg.<name>", "optimizer.exp_avg_sq.<name>"), "optimizer.step" (i64)
 * and the loss scaler ("amp.loss_scale" f32, "amp.good_steps" i64), which the reference's
 * loader skips as unknown names; the reference saves no optimizer state (the argument is
 * unused at checkpoint.cpp:34).  Loading skips unknown names and fails on a shape or dtype
 * mismatch, as the reference does; *has_optimizer reports whether AdamW state was restored.
 * description: up to desc_cap bytes including the terminating NUL. */
int aic_lm_save_checkpoint(aic_lm* lm, const char* path, int64_t step, int64_t epoch, float best_val_loss,
                           const char* description, int with_optimizer);
int aic_lm_load_checkpoint(aic_lm* lm, const char* path, int64_t* step, int64_t* epoch, float* best_val_loss,
                           char* description, int desc_cap, int* has_optimizer);

/* ---------------------------------------------------------------- token data -------- */
/* BinaryTokenDataset (include/data/dataset.hpp, src/data/dataset.cpp:155-219): a file of raw
 * int64 tokens (memory-mapped) or an in-memory copy; sample i is tokens[i*stride, +seq_len]
 * with targets shifted by one token; size = (total - 1 - seq_len) / stride + 1 (0 when
 * total < seq_len + 1); stride <= 0 means seq_len.  get_item writes seq_len tokens to each
 * (host) output, either may be NULL. */
typedef struct aic_token_dataset aic_token_dataset;
int aic_dataset_open(const char* path, int64_t seq_len, int64_t stride, aic_token_dataset** out);
int aic_dataset_from_tokens(const int64_t* tokens, int64_t n, int64_t seq_len, int64_t stride,
                            aic_token_dataset** out);
int aic_dataset_destroy(aic_token_dataset* ds);
int64_t aic_dataset_size(const aic_token_dataset* ds);
int64_t aic_dataset_total_tokens(const aic_token_dataset* ds);
int aic_dataset_get_item(const aic_token_dataset* ds, int64_t idx, int64_t* input, int64_t* target);
/* BinaryTokenDataset::write_binary_file (src/data/dataset.cpp:207-217). */
int aic_dataset_write_binary_file(const char* path, const int64_t* tokens, int64_t n);
/* DataLoader (include/data/dataloader.hpp, src/data/dataloader.cpp:12-78): batches of
 * batch_size samples (the last one smaller unless drop_last), the sample order shuffled with
 * std::shuffle over a std::mt19937_64(seed) at creation and at every reset (the reference's
 * order exactly, with the same standard library).  The loader keeps the dataset alive.
 * next_host: [b, seq_len] int64 inputs / targets in host memory; *actual_batch = b.
 * next_device: the same batch into device buffers, ordered on `stream`; with resident = 1 the
 * token array is copied to the device once (first call) and each batch is one gather kernel
 * over its window starts, otherwise the batch is assembled in pinned host memory and copied
 * asynchronously (two staging buffers, each reused after its copy completed). */
typedef struct aic_token_loader aic_token_loader;
int aic_loader_create(aic_token_dataset* ds, int64_t batch_size, int shuffle, int drop_last, uint64_t seed,
                      int resident, aic_token_loader** out);
int aic_loader_destroy(aic_token_loader* loader);
int64_t aic_loader_num_batches(const aic_token_loader* loader);
int aic_loader_has_next(const aic_token_loader* loader);
int aic_loader_reset(aic_token_loader* loader);
int aic_loader_next_host(aic_token_loader* loader, int64_t* inputs, int64_t* targets, int64_t* actual_batch);
int aic_loader_next_device(aic_token_loader* loader, int64_t* inputs, int64_t* targets, int64_t* actual_batch,
                           aic_stream stream);

/* ---------------------------------------------------------------- telemetry --------- */
/* TelemetryTracker (include/autonomous/telemetry.hpp, src/autonomous/telemetry.cpp:126-275):
 * EMAs of the loss (alpha_short, alpha_long) and gradient norm, the population variance of the
 * finite losses in the window, TFLOP/s = 6 P tokens/s, host (and, for device_index >= 0, GPU)
 * memory, and the anomaly of the step: non-finite loss (1) or gradient (2); else divergence
 * (3: loss above 1.4x the long EMA for 3 consecutive steps, from the third record), gradient
 * explosion (4: above 4x the gradient EMA, from the fifth record), vanishing gradient (5: below
 * 1e-7), GPU memory critical (6: under 8% free).  The is_* queries take the reference's
 * default thresholds when their arguments are <= 0. */
typedef struct aic_telemetry aic_telemetry;
typedef struct {
    int64_t step;
    float loss, loss_ema_short, loss_ema_long, loss_variance, grad_norm, grad_norm_ema, lr, tokens_per_sec,
        estimated_tflops;
    uint64_t host_total_bytes, host_free_bytes, gpu_total_bytes, gpu_free_bytes;
    int32_t anomaly;
    int32_t pad;
} aic_telemetry_snapshot;
int aic_telemetry_create(int64_t window, float alpha_short, float alpha_long, aic_telemetry** out);
int aic_telemetry_destroy(aic_telemetry* t);
int aic_telemetry_record(aic_telemetry* t, int64_t step, float loss, float grad_norm, float lr, float tokens_per_sec,
                         double step_seconds, int64_t total_tokens, int64_t model_params, int device_index,
                         aic_telemetry_snapshot* out);
int64_t aic_telemetry_count(const aic_telemetry* t);
int aic_telemetry_is_nan_or_inf(const aic_telemetry* t);
int aic_telemetry_is_diverging(const aic_telemetry* t, float threshold_ratio, int min_consecutive);
int aic_telemetry_is_gradient_exploding(const aic_telemetry* t, float spike_factor);
int aic_telemetry_is_gradient_vanishing(const aic_telemetry* t, float min_norm);
int aic_telemetry_reset(aic_telemetry* t);
/* The snapshot as one JSON object (the reference's TelemetrySnapshot::to_json fields plus the
 * memory counters and the anomaly name); buf of cap bytes, NUL-terminated. */
int aic_telemetry_latest_json(const aic_telemetry* t, char* buf, int cap);

/* ---------------------------------------------------------------- synthetic data ---- */
/* Host-side counter-based generators (splitmix64), shared by the tests and the bench.
 * Uniform ids in [0, vocab); Zipf(s) ids (P(k) ~ k^-s over ranks k = 1..vocab, id = k-1,
 * inverse-CDF); N(mean, std) floats via Box-Muller. */
int aic_synth_uniform_ids(uint64_t seed, int64_t n, int64_t vocab, int64_t* out_host);
int aic_synth_zipf_ids(uint64_t seed, int64_t n, int64_t vocab, double s, int64_t* out_host);
int aic_synth_normal(uint64_t seed, int64_t n, float mean, float std, float* out_host);

#ifdef __cplusplus
}
#endif
#endif
