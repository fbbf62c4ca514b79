/*
 * aic_oracle.h -- CPU restatement of the AutonomousAICore TransformerLM training step.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (autonomousaicore_amd/) links,
 * imports or calls this library.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker or as the timed CPU
 * baseline, never as the measured GPU path.
 *
 * Every function restates the reference's CPU algorithm (fp32 storage, fp32 GEMM with
 * the AVX2 4x16 FMA microkernel, double-precision reductions) and cites the reference
 * file:line it follows.  Paths are relative to /root/reference/AutonomousAICore/.
 *
 * Pinning (what checks each function against something other than itself):
 *   orc_gemm              reference known answers (tests/unit/test_matmul.cpp:17-68)
 *                         + numpy float64 matmul on random inputs
 *   orc_rmsnorm_*         unit-RMS invariant (tests/unit/test_nn.cpp:58-81)
 *                         + torch.nn.functional.rms_norm float64 fwd/autograd bwd
 *   orc_rope_*            norm preservation + start_pos offset (tests/unit/test_nn.cpp:83-112),
 *                         pos 0 == identity, bwd == inverse rotation, adjoint identity
 *   orc_attention_*       torch scaled_dot_product_attention(is_causal) float64 + autograd
 *   orc_flash_*           torch SDPA float64 + autograd under the mask of the reference's test
 *                         (tests/unit/test_flash_attention.cpp:37-60), Sq != Sk both ways,
 *                         logsumexp, o[0] == v[0], unseen keys get zero gradients
 *   orc_swiglu_*          closed form silu(g)*u + torch autograd float64
 *   orc_ce_*              0.407606 known answer (tests/unit/test_optim.cpp:16-36),
 *                         +-1000 stability (:38-65), ignore_index zero rows (:101-129),
 *                         torch cross_entropy float64 + autograd; soft targets: torch
 *                         cross_entropy with probabilities, one-hot rows == index targets
 *   orc_embedding_*       gather bit-equal + scatter counts (tests/unit/test_model.cpp:15-48)
 *   orc_adamw             0.989 one-step answer (tests/unit/test_optim.cpp:209-237)
 *                         + torch.optim.AdamW float64
 *   orc_clip_grad_norm    sqrt(91) -> 5 (tests/unit/test_optim.cpp:191-207)
 *   orc_scaler_*          sequences of tests/unit/test_amp.cpp:56-142
 *   orc_moe_*             brute-force top-k, routing invariants (tests/unit/test_moe.cpp),
 *                         float64 autograd restatement of src/nn/moe.cpp
 *   orc_int4_*            exhaustive 16 nibble values and known bytes, half-away rounding,
 *                         packing count / compression / cosine (tests/unit/test_quantization.cpp:47-67),
 *                         |deq - x| <= s/2, byte idempotence; fp16 scales vs numpy float16
 *   orc_lora_*            B = 0 identity (tests/unit/test_lora.cpp:58-73), merge == unmerged
 *                         forward (:107-143), torch float64 autograd
 *   orc_binary/unary/...  reference known answers (tests/unit/test_ops.cpp, test_tensor.cpp:45-98,
 *                         test_shape.cpp:49-72), numpy broadcasting / as_strided / float64
 *                         reductions / float16 casts, torch bfloat16 casts
 *   orc_lm_step           whole step vs an independent torch float64 model built from
 *                         library routines (F.embedding, F.linear, F.rms_norm, SDPA,
 *                         F.silu, F.cross_entropy, clip_grad_norm_, torch.optim.AdamW)
 * The reference itself cannot be compiled here (include/tensor/tensor.hpp:135 is rejected
 * by g++ 11 and clang 22), so no function is pinned against a reference binary.
 */
#ifndef AIC_ORACLE_H
#define AIC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- threading of the GEMM row split (src/ops/cpu_gemm.cpp:143-175: min(hw, 24)) ---- */
void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- GEMM: C[M,N] = A[M,K] . B[K,N], all row-major contiguous (src/ops/cpu_gemm.cpp:119-177) ---- */
void orc_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K);

/* Linear y[T,out] = x[T,in] . W[out,in]^T, run per batch of S rows (include/nn/linear.hpp:31-41,
 * src/ops/cpu_gemm.cpp:180-254). */
void orc_linear_fwd(const float* x, const float* W, float* y, int64_t B, int64_t S, int64_t in, int64_t out);
/* MatMulBackward (src/autograd/functions.cpp:254-273): dx = dy . W ; dW = sum_b x_b^T dy_b
 * (batch sum in double, src/ops/cpu_ops.cpp:195-262).  Either output may be NULL. */
void orc_linear_bwd(const float* x, const float* W, const float* dy, float* dx, float* dW,
                    int64_t B, int64_t S, int64_t in, int64_t out);

/* ---- RMSNorm (include/nn/rms_norm.hpp:18-34) ---- */
void orc_rmsnorm_fwd(const float* x, const float* w, float* y, float* rms, int64_t rows, int64_t d, float eps);
/* dx = dy*w/rms - x * sum(dy*w*x) / (d*rms^3); dw += sum_rows dy*x/rms (double). */
void orc_rmsnorm_bwd(const float* dy, const float* x, const float* w, const float* rms,
                     float* dx, float* dw, int64_t rows, int64_t d);

/* ---- RoPE, half-split, tables built like include/nn/rope.hpp:122-144 ---- */
void orc_rope_tables(float* cos_t, float* sin_t, int64_t max_seq, int64_t hd, float base);
/* x laid out [B, S, H, hd] (the [B,S,d] projection output); rotated in place,
 * position of row s is start_pos + s (include/nn/rope.hpp:66-112). */
void orc_rope_fwd(float* x, const float* cos_t, const float* sin_t, int64_t B, int64_t S, int64_t H,
                  int64_t hd, int64_t start_pos);
/* Adjoint rotation (include/nn/rope.hpp:23-39), in place. */
void orc_rope_bwd(float* g, const float* cos_t, const float* sin_t, int64_t B, int64_t S, int64_t H,
                  int64_t hd, int64_t start_pos);

/* ---- causal self-attention core, default (materialised) path (include/nn/attention.hpp:84-119) ----
 * q, k, v, o in [B, S, H, hd] layout.  E ([B,H,S,S]) receives exp(score - rowmax) and
 * rowsum ([B,H,S]) the float row sums, which the backward needs (softmax = E / rowsum,
 * src/ops/ops.cpp:460-471).  Both may be NULL when no backward follows. */
void orc_attention_fwd(const float* q, const float* k, const float* v, float* o, float* E, float* rowsum,
                       int64_t B, int64_t S, int64_t H, int64_t hd, int causal);
/* Backward of the same graph: matmul, mul(scale), add(mask), max/sub/exp/sum/div, matmul
 * (src/autograd/functions.cpp:60-78 Div, :150-170 Exp/Sum, :254-273 MatMul). */
void orc_attention_bwd(const float* q, const float* k, const float* v, const float* E, const float* rowsum,
                       const float* dout, float* dq, float* dk, float* dv, int64_t B, int64_t S, int64_t H,
                       int64_t hd);

/* ---- flash attention, CPU path (src/ops/flash_attention.cpp:32-260) ----
 * q, o [BH, Sq, D], k, v [BH, Sk, D], lse [BH, Sq] (the reference's [B, H, S, D] with BH = B*H).
 * Online softmax over key blocks of 32; causal: query r sees keys c <= r; a row with no key
 * gets o = 0 and lse = 0.  The backward accumulates into dq, dk, dv (zero them first). */
void orc_flash_fwd(const float* q, const float* k, const float* v, float* o, float* lse, int64_t BH, int64_t Sq,
                   int64_t Sk, int64_t D, int causal, float scale);
void orc_flash_bwd(const float* q, const float* k, const float* v, const float* o, const float* dout,
                   const float* lse, float* dq, float* dk, float* dv, int64_t BH, int64_t Sq, int64_t Sk, int64_t D,
                   int causal, float scale);

/* ---- SwiGLU activation h = silu(g) * u (include/nn/swiglu.hpp:21-33, src/ops/cpu_ops.cpp:143-146) ---- */
void orc_swiglu_fwd(const float* g, const float* u, float* h, int64_t n);
/* SiluBackward s*(1+x*(1-s)) (src/autograd/functions.cpp:167-175) and MulBackward. */
void orc_swiglu_bwd(const float* g, const float* u, const float* dh, float* dg, float* du, int64_t n);

/* ---- cross-entropy with index targets (src/loss/cross_entropy.cpp:149-290) ----
 * Returns the reduced loss ("mean" over valid rows); losses/lse may be NULL. */
float orc_ce_fwd(const float* logits, const int64_t* targets, int64_t N, int64_t C, int64_t ignore_index,
                 float* losses, float* lse, int64_t* valid_count);
/* grad = (exp(z - lse) - onehot) * g / valid (src/loss/cross_entropy.cpp:77-127). */
void orc_ce_bwd(const float* logits, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                int64_t ignore_index, int64_t valid_count, float g, float* dlogits);
/* The same for the reductions "mean" (g[0] / valid_count), "sum" (g[0]) and "none" (g[i]);
 * g may be NULL (1) (src/loss/cross_entropy.cpp:86-105). */
enum { ORC_CE_MEAN = 0, ORC_CE_SUM = 1, ORC_CE_NONE = 2 };
void orc_ce_bwd_reduction(const float* logits, const int64_t* targets, const float* lse, int64_t N, int64_t C,
                          int64_t ignore_index, int reduction, int64_t valid_count, const float* g, float* dlogits);

/* Soft (distribution) targets y [N, C]: losses[i] = lse_i - sum_j y_ij z_ij, every row counted;
 * returns the "mean" over N (src/loss/cross_entropy.cpp:240-248, 262-270).  The backward writes
 * (exp(z - lse) - y) * scale_i, scale_i = g[i] when per_row (g NULL: 1), else g[0] / divisor
 * (src/loss/cross_entropy.cpp:86-105, 120-125). */
float orc_ce_fwd_soft(const float* logits, const float* y, int64_t N, int64_t C, float* losses, float* lse);
void orc_ce_bwd_soft(const float* logits, const float* y, const float* lse, int64_t N, int64_t C, const float* g,
                     int per_row, float divisor, float* dlogits);

/* ---- Embedding (src/nn/embedding.cpp:96-156, :26-82) ---- */
void orc_embedding_fwd(const int64_t* ids, const float* W, float* out, int64_t N, int64_t D, int64_t V);
void orc_embedding_bwd(const int64_t* ids, const float* dout, float* dW, int64_t N, int64_t D, int64_t V);

/* ---- optimizer tail ---- */
/* AdamW::step for one tensor (src/optim/adamw.cpp:14-90); step = the incremented count. */
void orc_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
               float eps, float wd, int64_t step);
/* clip_grad_norm_ (src/optim/clip_grad.cpp:11-53) over `count` gradient buffers. */
float orc_clip_grad_norm(float* const* grads, const int64_t* sizes, int64_t count, float max_norm);

/* DynamicLossScaler (src/train/amp.cpp:50-152). */
typedef struct {
    float initial_scale, growth_factor, backoff_factor;
    int growth_interval;
    float min_scale, max_scale;
    float scale;
    int good_steps, skipped_steps;
} orc_scaler;
void orc_scaler_init(orc_scaler* s, float initial_scale, float growth_factor, float backoff_factor,
                     int growth_interval, float min_scale, float max_scale);
/* Returns 1 and unscales in place if every gradient is finite, else backs off and returns 0. */
int orc_scaler_unscale_and_update(orc_scaler* s, float* const* grads, const int64_t* sizes, int64_t count);

/* ---- whole TransformerLM training step ----
 * Parameter layout of `params` (and of grads / m / v), one flat float buffer:
 *   tok_embeddings.weight [V, d]
 *   for each layer l: attn.q_proj [d,d], attn.k_proj [d,d], attn.v_proj [d,d], attn.out_proj [d,d],
 *                     ffn.gate_proj [f,d], ffn.up_proj [f,d], ffn.down_proj [d,f],
 *                     norm1.weight [d], norm2.weight [d]
 *   norm.weight [d]
 *   lm_head.weight [V, d]      (absent when tied: the head reuses tok_embeddings.weight)
 * With n_experts = E > 0 (MoETransformerLM, src/models/moe_transformer_lm.cpp) the three ffn
 * tensors of a layer are replaced by moe.router.gate.weight [E,d] and, for each expert e,
 * moe.experts.e.gate_proj [f,d], up_proj [f,d], down_proj [d,f]; the loss is cross_entropy +
 * total_aux_loss (the layers' aux losses added in layer order).
 */
typedef struct {
    int64_t vocab, d_model, n_layers, n_heads, d_ffn, max_seq_len;
    float norm_eps, rope_base;
    int tied;
    int64_t n_experts, top_k;
    float aux_coef;
} orc_lm_config;

typedef struct {
    float lr, beta1, beta2, eps, weight_decay;
    float max_grad_norm;   /* <= 0: no clipping */
    int use_scaler;        /* 1: loss scaling as Trainer::step with AMP (src/train/trainer.cpp:37-118) */
    int do_update;         /* 0: stop after backward (grads only) */
} orc_train_opts;

typedef struct {
    float loss;
    float grad_norm;       /* pre-clip global L2 norm of the (unscaled) gradients */
    int found_inf;         /* scaler found a non-finite gradient; the update was skipped */
    float loss_scale_used;
    double t_embed, t_blocks_fwd, t_head_fwd, t_loss, t_head_bwd, t_blocks_bwd, t_embed_bwd, t_optim; /* seconds */
    float aux_loss;        /* MoE: total_aux_loss (included in loss) */
} orc_step_result;

int64_t orc_lm_num_params(const orc_lm_config* cfg);
/* Loss only (no grad), used for finite-difference checks. */
float orc_lm_loss(const orc_lm_config* cfg, const float* params, const int64_t* ids, const int64_t* targets,
                  int64_t B, int64_t S);
/* One step: forward, cross_entropy(mean, ignore -100), backward, [scaler], clip, AdamW.
 * grads receives the gradients seen by the optimizer (unscaled, post-clip).
 * m/v/step_count: AdamW state; scaler may be NULL when opts->use_scaler == 0. */
/* Forward only: logits [B*S, V] of TransformerLM::forward. */
int orc_lm_logits(const orc_lm_config* cfg, const float* params, const int64_t* ids, int64_t B, int64_t S,
                  float* logits);
int orc_lm_step(const orc_lm_config* cfg, float* params, float* grads, float* m, float* v, int64_t* step_count,
                const int64_t* ids, const int64_t* targets, int64_t B, int64_t S, const orc_train_opts* opts,
                orc_scaler* scaler, orc_step_result* res);

/* QLoRA TransformerLM step (LoRAAdapter::apply over QuantizedLinear::from_linear,
 * src/nn/lora.cpp:116-175, src/nn/quantization.cpp:669-679; dense FFN only).  base: the dense
 * parameters (orc_lm_num_params, frozen); the seven projections of each layer enter as their INT4
 * round trip (groups of G, fp16 scales).  lora: orc_qlora_num_params adapters, per layer A of
 * q, k, v [r,d]; B of q, k, v [d,r]; A, B of out_proj; A of gate, up [r,d]; B of gate, up
 * [f,r]; A of down [r,f]; B of down [d,r]; scaling alpha / r.  grads/m/v: adapter-sized. */
int64_t orc_qlora_num_params(const orc_lm_config* cfg, int64_t r);
int orc_qlora_dequantize_base(const orc_lm_config* cfg, int64_t G, float* params);
int orc_qlora_step(const orc_lm_config* cfg, int64_t r, float alpha, int64_t G, const float* base, float* lora,
                   float* grads, float* m, float* v, int64_t* step_count, const int64_t* ids, const int64_t* targets,
                   int64_t B, int64_t S, const orc_train_opts* opts, orc_scaler* scaler, orc_step_result* res);

/* ---- Mixture of experts (src/nn/moe.cpp) ---- */
/* Router on gate logits [T,E] (moe.cpp:33-129) plus the gate normalisation of MoELayer::forward
 * (moe.cpp:170-204); top-k ties go to the lower expert index.  Any output may be NULL. */
void orc_moe_route(const float* logits, int64_t T, int64_t E, int64_t k, float aux_coef, int64_t* idx,
                   float* rweights, float* gates, float* probs, int64_t* counts, float* mean_probs, float* aux);
/* MoELayer::forward on h [T,d]: router wr [E,d]; experts wg/wu [E,f,d], wd [E,d,f]. */
void orc_moe_ffn_fwd(const float* h, const float* wr, const float* wg, const float* wu, const float* wd, int64_t T,
                     int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, float* y, float* aux, int64_t* idx,
                     float* gates);
/* Test control of the MoE LM step's routing (orc_lm_step, orc_lm_loss, orc_lm_logits): with
 * forced != NULL ([n_layers][T][top_k], k distinct experts per token) every layer uses that top-k
 * selection instead of its router's (probabilities, gates, counts and aux follow from it); with
 * out != NULL the selections the forward used are written there.  Stays set until called again
 * (NULL, NULL). */
void orc_moe_set_routing(const int64_t* forced, int64_t* out);
/* Its backward for dL/dy and dL/daux; gradients are added into dh, dwr, dwg, dwu, dwd (E <= 256). */
void orc_moe_ffn_bwd(const float* h, const float* wr, const float* wg, const float* wu, const float* wd, int64_t T,
                     int64_t d, int64_t f, int64_t E, int64_t k, float aux_coef, const float* dy, float daux, float* dh,
                     float* dwr, float* dwg, float* dwu, float* dwd);

/* ---- INT4 symmetric quantization (src/nn/quantization.cpp) ---- */
/* IEEE binary32 <-> binary16 (round to nearest even; subnormals kept). */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
/* QuantizedTensor::quantize, INT4_SYMMETRIC (quantization.cpp:197-295): groups of G consecutive
 * elements of the flat row-major x[n] (G <= 0 or G > n: one group); s = max(absmax/7, 1e-8);
 * q = clamp(round_half_away(x/s), -7, 7); packed[(n+1)/2] holds element 2i in the low nibble
 * (include/nn/quantization.hpp:41-44).  scales[ceil(n/G)]: fp32, or (scale_f16) the fp16 bits
 * of s; q always uses the fp32 s, so the packed bytes equal the reference's either way.
 * Returns 0, 1 for n < 0, 2 for an odd G with more than one group. */
int orc_int4_quantize(const float* x, int64_t n, int64_t G, int scale_f16, uint8_t* packed, void* scales);
/* QuantizedTensor::dequantize (quantization.cpp:433-443): out[i] = q_i * s_{i/G}. */
int orc_int4_dequantize(const uint8_t* packed, const void* scales, int scale_f16, int64_t n, int64_t G, float* out);
/* launch_dequantize_int4 (src/cuda/cuda_quantize.cu:54-94): signed or unsigned nibbles, optional fp32 zero
 * points, fp32 scales; out = (val - zp[g]) * s[g]. */
int orc_int4_dequantize_zp(const uint8_t* packed, const float* scales, const float* zp, int is_signed, int64_t n,
                           int64_t G, float* out);

/* ---- LoRA (src/nn/lora.cpp) ---- */
/* LoRALinear::forward (lora.cpp:75-93) on base weight W [out,in] (a Linear, or the dequantized
 * INT4 weight of QuantizedLinear::forward, quantization.cpp:669-679), A [r,in], Bm [out,r]:
 * y = x W^T + ((x A^T) Bm^T) * scaling, each product per batch of S rows.  xa [T,r] may be NULL. */
void orc_lora_fwd(const float* x, const float* W, const float* A, const float* Bm, float scaling, int64_t Bt,
                  int64_t S, int64_t in, int64_t out, int64_t r, float* y, float* xa);
/* Its backward with W frozen (lora.cpp:54-56): dl = dy*scaling; dxa = dl Bm; dBm += dl^T xa;
 * dA += dxa^T x; dx = dy W + dxa A (overwritten).  Any output may be NULL. */
void orc_lora_bwd(const float* x, const float* W, const float* A, const float* Bm, float scaling, const float* dy,
                  int64_t Bt, int64_t S, int64_t in, int64_t out, int64_t r, float* dx, float* dA, float* dB);
/* LoRALinear::merge / unmerge (lora.cpp:95-108): W = W +- (Bm A) * scaling (sign >= 0: merge). */
void orc_lora_merge(float* W, const float* A, const float* Bm, float scaling, int64_t in, int64_t out, int64_t r,
                    int sign);

/* ---- Tensor primitives (fp32 compute; src/ops/cpu_ops.cpp, src/tensor/tensor.cpp) ---- */
/* Shape::broadcast (src/core/shape.cpp:138-166): output rank, or -1 if incompatible. */
int orc_broadcast_shape(const int64_t* a, int ra, const int64_t* b, int rb, int64_t* out);
/* Tensor::clone of a strided view (src/tensor/tensor.cpp:255-297); ndim <= 16. */
void orc_strided_copy(const void* src, int64_t offset, int ndim, const int64_t* shape, const int64_t* strides,
                      int64_t elem_size, void* dst);
/* Tensor::to(DType) (src/tensor/tensor.cpp:359-410); codes 0 f32, 1 f16, 2 bf16, 3 i32, 4 i64.
 * Returns 1 for a pair the reference does not implement. */
int orc_cast(const void* src, int from, void* dst, int to, int64_t n);
/* binary_broadcast_cpu (src/ops/cpu_ops.cpp:14-60): op 0 add, 1 sub, 2 mul, 3 div. */
int orc_binary(int op, const float* a, int64_t a_off, const int64_t* a_shape, const int64_t* a_strides, int ra,
               const float* b, int64_t b_off, const int64_t* b_shape, const int64_t* b_strides, int rb, float* out);
/* unary_cpu (src/ops/cpu_ops.cpp:105-146): 0 neg, 1 abs, 2 exp, 3 log, 4 sqrt, 5 tanh, 6 sigmoid,
 * 7 gelu, 8 silu. */
void orc_unary(int op, const float* x, float* y, int64_t n);
/* sum / mean / max / min over all elements (src/ops/cpu_ops.cpp:151-197): op 0..3. */
float orc_reduce_all(int op, const float* x, int64_t n);
/* reduce_dim_cpu (src/ops/cpu_ops.cpp:203-271) of a contiguous tensor along dim. */
void orc_reduce_dim(int op, const float* x, int ndim, const int64_t* shape, int dim, float* out);
/* cat (src/ops/ops.cpp:473-530) of contiguous [outer, mid_i, inner] inputs. */
void orc_cat(const void* const* srcs, const int64_t* mids, int count, int64_t outer, int64_t inner, int64_t elem_size,
             void* dst);
/* reduce_gradient_for_broadcast (src/autograd/functions.cpp:10-41). */
int orc_sum_to_shape(const float* g, int ndim, const int64_t* shape, int tr, const int64_t* target, float* out);

#ifdef __cplusplus
}
#endif
#endif
