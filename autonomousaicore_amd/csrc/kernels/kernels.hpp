// Host launchers of the non-GEMM kernels.  All take explicit leading dimensions (elements),
// enqueue on `s` and throw aic::Error on invalid arguments or launch failure.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../runtime/dtype.hpp"

namespace aic::hip {

// RMSNorm (norm.hip)
void rmsnorm_fwd(const void* x, int64_t ldx, const float* w, void* y, int64_t ldy, float* rms, int64_t rows,
                 int64_t dim, float eps, DType dt, hipStream_t s);
void rmsnorm_bwd(const void* dy, int64_t lddy, const void* x, int64_t ldx, const float* w, const float* rms,
                 const void* dres, int64_t ldres, void* dx, int64_t lddx, float* dw, bool accumulate, int64_t rows,
                 int64_t dim, DType dt, hipStream_t s);
// rmsnorm_bwd whose weight gradient is left as rmsnorm_bwd_part_rows(rows) partial rows of dim
// floats in `part` (dim % 8 == 0); rmsnorm_dw_reduce later overwrites each dws[t] with the sum
// of parts[t]'s rows in rmsnorm_bwd's own order (bit-identical to it), all norms in one launch.
int64_t rmsnorm_bwd_part_rows(int64_t rows);
void rmsnorm_bwd_deferred(const void* dy, int64_t lddy, const void* x, int64_t ldx, const float* w, const float* rms,
                          const void* dres, int64_t ldres, void* dx, int64_t lddx, float* part, int64_t rows,
                          int64_t dim, DType dt, hipStream_t s);
void rmsnorm_dw_reduce(const float* const* parts, float* const* dws, int count, int64_t rows, int64_t dim,
                       hipStream_t s);

// RoPE (rope.hip)
void rope(void* x, int64_t ld, int64_t B, int64_t S, int64_t heads, int64_t hd, int64_t start_pos, const float* cos_t,
          const float* sin_t, bool inverse, DType dt, hipStream_t s);
void rope_tables_host(float* cos_t, float* sin_t, int64_t max_seq, int64_t hd, float base);

// SwiGLU activation (swiglu.hip)
void swiglu_fwd(const void* g, const void* u, int64_t ld_gu, void* h, int64_t ld_h, int64_t T, int64_t f, DType dt,
                hipStream_t s);
void swiglu_bwd(const void* g, const void* u, int64_t ld_gu, const void* dh, int64_t ld_h, void* dg, void* du,
                int64_t ld_d, int64_t T, int64_t f, DType dt, hipStream_t s);

// Cross-entropy (loss.hip)
void ce_fwd(const void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
            float* losses, float* lse, float* loss_mean, int64_t* valid, DType dt, hipStream_t s);
void ce_bwd(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N, int64_t C,
            int64_t ignore_index, const float* grad, const int64_t* valid, void* dlogits, int64_t ld_d, DType dt,
            hipStream_t s);
void ce_bwd_rows(const void* logits, int64_t ld, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                 int64_t ignore_index, const float* grad, int per_row, float divisor, void* dlogits, int64_t ld_d,
                 DType dt, hipStream_t s);
// Soft targets y [N, C] fp32 (leading dimension ldy): row losses lse - sum_j y_j z_j, every row
// valid (loss_mean over N); the backward writes (softmax - y) times the row weight of ce_bwd_rows.
void ce_fwd_soft(const void* logits, int64_t ld, const float* y, int64_t ldy, int64_t N, int64_t C, float* losses,
                 float* lse, float* loss_mean, DType dt, hipStream_t s);
void ce_bwd_soft(const void* logits, int64_t ld, const float* y, int64_t ldy, const float* lse, int64_t N, int64_t C,
                 const float* grad, int per_row, float divisor, void* dlogits, int64_t ld_d, DType dt, hipStream_t s);
// Forward and backward in one pass: ce_fwd's outputs (valid required) and the logits overwritten by
// ce_bwd's gradient with grad (device scalar, null: 1) over the valid rows.
void ce_fwd_bwd(void* logits, int64_t ld, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
                float* losses, float* lse, float* loss_mean, int64_t* valid, const float* grad, DType dt,
                hipStream_t s);

// Embedding (embedding.hip)
void embed_fwd(const int64_t* ids, int64_t N, const void* W, int64_t V, int64_t D, void* out, DType dt, hipStream_t s);
void embed_bwd(const int64_t* ids, int64_t N, const void* dout, int64_t V, int64_t D, float* dW, bool accumulate,
               DType dt, hipStream_t s);

// Mixture of experts (moe.hip).  Expert row blocks start at multiples of 64 rows.
int64_t moe_max_rows(int64_t T, int64_t E, int64_t k);
void moe_route(const float* logits, int64_t T, int64_t E, int64_t k, float aux_coef, int64_t* idx, float* gsel,
               float* probs, float* rweights, int64_t* counts, float* mean_probs, float* aux, hipStream_t s);
void moe_permute(const int64_t* idx, const int64_t* counts, int64_t T, int64_t k, int64_t E, int64_t* offsets,
                 int* dst_row, int* src_ent, hipStream_t s);
void moe_gather(const void* x, int64_t ldx, const int* src_ent, int64_t k, int64_t rows, int64_t d, void* xp, DType dt,
                hipStream_t s);
void moe_combine(const void* ye, const int64_t* idx, const int* dst_row, const float* gsel, int64_t T, int64_t k,
                 int64_t d, const void* R, int64_t ldr, void* out, int64_t ldo, DType dt, hipStream_t s);
void moe_combine_bwd(const void* dout, int64_t ldo, const void* ye, const int* src_ent, const float* gsel, int64_t rows,
                     int64_t k, int64_t d, void* dye, float* dgsel, DType dt, hipStream_t s);
// With router_dlogits (fp32 [T, E]) and router_w ([E, d], dtype dt) the router's input gradient
// dlogits[t] . W_r is added to each token's sum in fp32 before the one rounding to dt.
void moe_scatter(const void* dxp, const int64_t* idx, const int* dst_row, int64_t T, int64_t k, int64_t d, void* dx,
                 int64_t ldx, bool accumulate, DType dt, hipStream_t s, const float* router_dlogits = nullptr,
                 const void* router_w = nullptr, int64_t E = 0);
// daux_scale (device, nullable) multiplies daux: the loss scale of an AMP step.
void moe_router_bwd(const float* probs, const int64_t* idx, const float* dgsel, const int64_t* counts, int64_t T,
                    int64_t E, int64_t k, float aux_coef, float daux, const float* daux_scale, float* dlogits,
                    hipStream_t s);
// *total = aux[0] + aux[1] + ... (layer order); *loss += *total.  MoETransformerLM::total_aux_loss.
void moe_aux_total(const float* aux, int64_t L, float* loss, float* total, hipStream_t s);

// INT4 symmetric quantization (int4.hip).  Scales are f32 or f16; the dequantized output f32 or
// bf16.  int4_group returns the effective group size (G <= 0 or G > n: n) and rejects an odd one.
int64_t int4_group(int64_t n, int64_t G);
void int4_quantize(const float* x, int64_t n, int64_t G, uint8_t* packed, void* scales, DType scale_t, hipStream_t s);
void int4_dequant(const uint8_t* packed, const void* scales, DType scale_t, int64_t n, int64_t G, void* out, DType out_t,
                  hipStream_t s);
// The CUDA launcher's general INT4 dequantization: zero points (or none), signed or unsigned
// nibbles, fp32 scales and output, any group size (<= 0: one group).
void int4_dequant_zp(const uint8_t* packed, const float* scales, const float* zp, bool is_signed, int64_t n,
                     int64_t G, float* out, hipStream_t s);

// Tensor primitives (tensor_ops.hip).  Views are (offset, rank <= 8, shape, strides) in elements;
// binary ops broadcast NumPy-style into a contiguous output.  op codes: binary 0 add, 1 sub,
// 2 mul, 3 div; unary 0 neg, 1 abs, 2 exp, 3 log, 4 sqrt, 5 tanh, 6 sigmoid, 7 gelu, 8 silu;
// reductions 0 sum, 1 mean, 2 max, 3 min.
void strided_copy(const void* src, int64_t offset, int ndim, const int64_t* shape, const int64_t* strides,
                  int64_t elem_size, void* dst, hipStream_t s);
void cast(const void* src, DType from, void* dst, DType to, int64_t n, hipStream_t s);
void binary(int op, const float* a, int64_t a_off, int ra, const int64_t* a_shape, const int64_t* a_strides,
            const float* b, int64_t b_off, int rb, const int64_t* b_shape, const int64_t* b_strides, float* out,
            hipStream_t s);
void unary(int op, const float* x, float* y, int64_t n, hipStream_t s);
void reduce_all(int op, const float* x, int64_t n, float* out, hipStream_t s);
void reduce_dim(int op, const float* x, int ndim, const int64_t* shape, int dim, float* out, hipStream_t s);
void cat(const void* const* srcs, const int64_t* mids, int count, int64_t outer, int64_t inner, int64_t elem_size,
         void* dst, hipStream_t s);
void sum_to_shape(const float* g, int ndim, const int64_t* shape, int tr, const int64_t* target, float* out,
                  hipStream_t s);

// Attention (attention.hip)
void attn_fwd(const void* q, const void* k, const void* v, int64_t ld_qkv, void* o, int64_t ld_o, float* lse,
              int64_t B, int64_t H, int64_t S, int64_t hd, bool causal, float scale, DType dt, hipStream_t s);
// rope_cos / rope_sin ([S][hd / 2] tables, positions 0..S-1 of each sequence): dq and dk leave
// with the half-split rotary embedding's adjoint applied (rope(..., inverse = true) fused).
void attn_bwd(const void* q, const void* k, const void* v, int64_t ld_qkv, const void* o, const void* dout,
              int64_t ld_o, const float* lse, void* dq, void* dk, void* dv, int64_t ld_d, int64_t B, int64_t H,
              int64_t S, int64_t hd, bool causal, float scale, DType dt, hipStream_t s,
              const float* rope_cos = nullptr, const float* rope_sin = nullptr);
// Queries and keys of different lengths Sq, Sk (causal: query r sees keys c <= r).
void attn_fwd_qk(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_k, void* o, int64_t ld_o,
                 float* lse, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t hd, bool causal, float scale,
                 DType dt, hipStream_t s);
void attn_bwd_qk(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_k, const void* o,
                 const void* dout, int64_t ld_o, const float* lse, void* dq, int64_t ld_dq, void* dk, void* dv,
                 int64_t ld_dkv, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t hd, bool causal, float scale,
                 DType dt, hipStream_t s);
// Queries of S_new new tokens (rows of q, [B*S_new] x ldq) at positions start_pos.. against a
// KV cache kc / vc ([B][cache_rows][ldkv], positions 0 .. start_pos+S_new-1 filled), causal.
void attn_cached(const void* q, int64_t ldq, const void* kc, const void* vc, int64_t ldkv, int64_t cache_rows, void* o,
                 int64_t ldo, int64_t B, int64_t H, int64_t S_new, int64_t start_pos, int64_t hd, float scale, DType dt,
                 hipStream_t s);

// Optimizer tail (optim.hip)
struct OptimCtl;  // = aic_optim_ctl (include/aic_hip.h)
void grad_sqnorm_multi(const float* const* grads, const int64_t* sizes, int count, double* sqnorm, int* nonfinite,
                       hipStream_t s);
void grad_sqnorm_multi_noalloc(const float* const* grads, const int64_t* sizes, int count, double* sqnorm,
                               int* nonfinite, hipStream_t s);
void scale_multi(float* const* grads, const int64_t* sizes, int count, const float* scale, hipStream_t s);
void optim_finalize(const double* sqnorm, const int* nonfinite, void* ctl, hipStream_t s);
// The gradient norm from partial slots written by the gradients' producers (GEMM epilogues,
// split-K reductions) plus these: sqnorm_partials writes sqnorm_k's partials of the tensors
// into pd / pn (sqnorm_slots(sizes, count) slots); sqnorm_reduce adds nslots slots in a fixed
// order (blocks of 4096, then one block over them; tmp_d / tmp_n hold sqnorm_reduce_tmp(nslots)
// entries) into *sqnorm and the OR of the flags into *nonfinite.
int64_t sqnorm_slots(const int64_t* sizes, int count);
void sqnorm_partials(const float* const* grads, const int64_t* sizes, int count, double* pd, int* pn, hipStream_t s);
void sqnorm_clear(double* pd, int* pn, int64_t nslots, hipStream_t s);  // every slot to 0
int64_t sqnorm_reduce_tmp(int64_t nslots);
void sqnorm_reduce(const double* pd, const int* pn, int64_t nslots, double* tmp_d, int* tmp_n, double* sqnorm,
                   int* nonfinite, hipStream_t s);
void adamw_multi(float* const* p, const float* const* g, float* const* m, float* const* v, void* const* p_bf16,
                 const int64_t* sizes, int count, float lr, float beta1, float beta2, float eps, float wd,
                 int64_t step, const void* ctl, hipStream_t s);
// Single-tensor AdamW with caller-computed bias corrections bc1 = 1 - beta1^t, bc2 = 1 - beta2^t.
void adamw_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2, float eps,
                float wd, float bc1, float bc2, hipStream_t s);
void cast_f32_bf16(const float* src, void* dst, int64_t n, hipStream_t s);
// Streaming probe (no reference counterpart): out_j = sum(in) + j, out_bf16 = bf16(sum(in)) over
// n fp32 elements, in the form of adamw_k; mixes: 1r, 1w, 1r1w, 2r1w, 4r3w + bf16.
void stream_probe(const float* const* in, int n_in, float* const* out, int n_out, void* out_bf16, float* sink,
                  int64_t n, bool nontemporal, hipStream_t s);
// Appends {step, loss, aux, grad_norm, loss scale, found_inf} (an aic_step_record) to a device
// ring of cap records; *count (device) counts all records ever appended.
void step_record(const float* loss, const float* aux, const void* ctl, const float* scale_used, void* ring,
                 int64_t* count, int cap, hipStream_t s);
void fill_normal(float* dst, int64_t n, uint64_t seed, uint64_t offset, float mean, float std, hipStream_t s);
void fill_const(float* dst, int64_t n, float v, hipStream_t s);

// LoRA adapter products in one pass over a bf16 operand Y [T, N] (leading dimension ldy) whose
// columns form N / n_seg segments of n_seg columns (n_seg % 256 == 0), each paired with r_seg
// (16, 32 or 48) columns of the small operands:
//   out1[t, g r_seg + j] = bf16(scale * sum_{n in segment g} Y[t, n] W(n, j))   when out1
//   out2(n, j) (+)= sum_t Y[t, n] Z[t, g(n) r_seg + j]                          when out2
// W(n, j) = W[n w_n + j w_j] with w_j == 1 (rows of j, w_n % 8 == 0) or w_n == 1 (rows of n,
// w_j % 8 == 0); out1 [T, ldo1] bf16; Z [T, ldz] bf16; out2 fp32 at out2 + n o2n + j o2j,
// overwritten or added to (accumulate).  bf16 inputs 16-byte aligned with ld % 8 == 0; out1
// 8-byte aligned with ldo1 % 4 == 0.
// Deterministic: partial sums in a fixed order, no atomics.
struct LoraSkinny {
    const void* Y = nullptr;
    int64_t ldy = 0, T = 0, N = 0, n_seg = 0, r_seg = 0;
    const void* W = nullptr;
    int64_t w_n = 0, w_j = 0;
    void* out1 = nullptr;
    int64_t ldo1 = 0;
    float scale = 1.0f;
    const void* Z = nullptr;
    int64_t ldz = 0;
    float* out2 = nullptr;
    int64_t o2n = 0, o2j = 0;
    bool accumulate = false;
};
bool lora_skinny_ok(const LoraSkinny& q);  // the shapes and layouts the kernel takes
void lora_skinny(const LoraSkinny& q, hipStream_t s);

}  // namespace aic::hip
