// TransformerLM training step on one GPU.
//
// Mirrors the reference's model and trainer API (models::TransformerLMConfig and
// TransformerLM, include/models/transformer_lm.hpp:19-76; optim::AdamWOptions,
// include/optim/adamw.hpp:12-18; train::DynamicLossScalerOptions,
// include/train/amp.hpp:34-41; Trainer::step, src/train/trainer.cpp:37-118) and runs the
// whole step -- forward, cross-entropy, backward, loss scaling, clip_grad_norm_ and AdamW --
// as one stream of fused HIP kernels:
//   * parameters, gradients and AdamW moments live in flat fp32 device arenas, one tensor
//     after another (q/k/v and gate/up adjacent so each pair/triple is one GEMM), with a
//     bf16 shadow copy of the weights refreshed by the AdamW kernel in AMP mode;
//   * the residual adds are fused into the out_proj/down_proj GEMM epilogues and the
//     residual-stream gradient adds into the RMSNorm backward;
//   * the loss scaler, the clip decision and the AdamW step count stay on the device, so a
//     step needs no host synchronisation (the reference syncs per parameter).
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <cstdint>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "../../../include/aic_hip.h"
#include "../runtime/checkpoint.hpp"
#include "../runtime/dtype.hpp"
#include "../runtime/profiler.hpp"
#include "moe_ffn.hpp"

namespace aic::models {

struct TransformerLMConfig {
    int64_t vocab_size = 320;
    int64_t hidden_dim = 128;
    int64_t num_layers = 4;
    int64_t num_heads = 4;
    int64_t intermediate_dim = 384;
    int64_t max_seq_len = 512;
    float rms_norm_eps = 1e-5f;
    float rope_theta = 10000.0f;
    bool tie_word_embeddings = false;
    DType compute = DType::Float32;  // Float32 (reference precision) or BFloat16 (AMP)
    // Mixture of experts (MoETransformerLMConfig, include/models/moe_transformer_lm.hpp): with
    // num_experts > 0 every FFN is a routed MoE layer of num_experts SwiGLU experts of
    // intermediate_dim, top_k per token, and the training loss adds each layer's aux loss.
    int64_t num_experts = 0;
    int64_t top_k = 2;
    float aux_loss_coef = 0.01f;
    // QLoRA (LoRAAdapter::apply over QuantizedLinear; src/nn/lora.cpp:116-175,
    // src/nn/quantization.cpp:669-679): lora_rank > 0 freezes every base weight, keeps the seven
    // projections of each layer as INT4-symmetric groups of quant_group elements with fp16
    // scales, and trains only the LoRA adapters (A [r, in], B [out, r], scaling alpha / r).
    int64_t lora_rank = 0;
    float lora_alpha = 32.0f;
    int64_t quant_group = 128;
};

struct AdamWOptions {
    float lr = 1e-3f, beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f, weight_decay = 0.01f;
};

struct DynamicLossScalerOptions {
    float initial_scale = 65536.0f, growth_factor = 2.0f, backoff_factor = 0.5f;
    int growth_interval = 1000;
    float min_scale = 1.0f, max_scale = 16777216.0f;
};

struct TrainOptions {
    AdamWOptions adamw;
    float max_grad_norm = 1.0f;
    bool use_loss_scaler = false;
    DynamicLossScalerOptions scaler;
};

struct ParamInfo {
    std::string name;
    std::vector<int64_t> shape;
    int64_t offset = 0;  // elements into the arena
    int64_t numel = 0;
};

struct StepStats {
    float loss = 0.0f;      // cross-entropy + the MoE aux losses (total_aux_loss)
    float aux_loss = 0.0f;  // sum of the MoE layers' aux losses (0 for a dense model)
    float grad_norm = 0.0f;
    bool found_inf = false;
    float loss_scale = 1.0f;
    int64_t step = 0;
};

// One token drawn from fp32 logits by TransformerLM::generate's rules (greedy, temperature,
// top-k, top-p, std::discrete_distribution over rng).
int64_t sample_token(const std::vector<float>& logits, float temperature, int top_k, float top_p,
                     std::mt19937_64& rng);

class TransformerLM {
public:
    TransformerLM(const TransformerLMConfig& cfg, const TrainOptions& opt);
    ~TransformerLM();
    TransformerLM(const TransformerLM&) = delete;
    TransformerLM& operator=(const TransformerLM&) = delete;

    const TransformerLMConfig& config() const { return cfg_; }
    // Trainable tensors (with QLoRA: the LoRA adapters) and the frozen base model's tensors (the
    // dense layout; the same list as params() without QLoRA).
    const std::vector<ParamInfo>& params() const { return params_; }
    const std::vector<ParamInfo>& base_params() const { return lora() ? base_ : params_; }
    int64_t arena_elems() const { return arena_; }
    int64_t num_params() const;
    hipStream_t stream() const { return stream_; }

    void set_params(const float* host);
    // QLoRA: the frozen base weights in base_params() order (packed, no padding); the seven
    // projections of each layer are then quantized to INT4 (QuantizedLinear::from_linear).
    void set_base_params(const float* host);
    void get_params(float* host) const;
    void get_base_params(float* host) const;
    void get_grads(float* host) const;
    // MoE: the top-k selection [T, top_k] of layer `layer` in the last forward, to host (at most
    // cap values; synchronises); returns T.
    int64_t moe_routing(int64_t layer, int64_t* host, int64_t cap) const;
    void get_adam_state(float* m, float* v, int64_t* step) const;
    void init_normal(uint64_t seed, float std, bool residual_scaling);

    // The reference's .aic checkpoint (save_checkpoint / load_checkpoint,
    // src/train/checkpoint.cpp:30-186): every parameter (with QLoRA the frozen base and the
    // adapters) as fp32 under its reference name, in Module::named_parameters() order.  With
    // with_optimizer the file also carries the AdamW moments ("optimizer.exp_avg.<name>",
    // "optimizer.exp_avg_sq.<name>"), the step count ("optimizer.step", i64) and the loss
    // scaler ("amp.loss_scale" f32, "amp.good_steps" i64) after the parameters -- entries the
    // reference's loader skips as unknown names.  load_checkpoint restores what the file holds
    // (unknown names are skipped, a shape or dtype mismatch throws) and reports in
    // *has_optimizer whether optimizer state was found.
    void save_checkpoint(const std::string& path, const CheckpointMeta& meta, bool with_optimizer);
    CheckpointMeta load_checkpoint(const std::string& path, bool* has_optimizer);

    // KV-cached inference (TransformerLM::forward_step and generate,
    // src/models/transformer_lm.cpp:64-233): ids are the device [B, S] int64 tokens at
    // positions start_pos .. start_pos + S - 1, whose keys and values join the cache (one cache
    // per layer, [B][max_seq_len][d] rows for K and for V, allocated on first use); logits
    // receives their fp32 logits [B * S, V] (device).  A call with start_pos == 0 starts a new
    // sequence (the whole prompt in one prefill).  generate() is the reference's loop for one
    // sequence: prefill, then one token per step, sampled on the host from the fp32 logits with
    // the reference's greedy / temperature / top-k / top-p rules and std::mt19937_64(seed).
    void forward_step(const int64_t* ids, int64_t B, int64_t S, int64_t start_pos, float* logits);
    std::vector<int64_t> generate(const std::vector<int64_t>& prompt, int64_t max_new_tokens, float temperature,
                                  int top_k, float top_p, int64_t eos_token_id, uint64_t seed);

    // Telemetry hooks: the records of the steps since the previous call (one synchronisation),
    // oldest first, at most cap; *dropped counts older records the ring overwrote.  snapshot()
    // keeps a device copy of the trainable parameters, AdamW moments and optimiser state;
    // restore() puts it back.
    int step_history(aic_step_record* out, int cap, int64_t* dropped);
    void snapshot();
    void restore();

    // ids/targets: device pointers to [B, S] int64.
    void train_step(const int64_t* ids, const int64_t* targets, int64_t B, int64_t S);
    float eval_loss(const int64_t* ids, const int64_t* targets, int64_t B, int64_t S);
    StepStats last_stats();
    void synchronize();

    // Per-kernel-class HIP-event timing of the following steps (resets when enabled).
    void set_profiling(bool on, uint32_t class_mask = 0xffffffffu) {
        prof_.set_mask(class_mask);
        prof_.enable(on);
    }
    std::vector<KernelClassStats> profile_stats() { return prof_.collect(); }

    // Whether the training step forms the gradient norm from partial sums written by the
    // gradients' producers (models with an untied LM head, dense or MoE) instead of a separate pass
    // over every gradient; on by default where the model allows it.  Returns whether it is used.
    bool set_fused_grad_norm(bool on) {
        sq_fold_on_ = on;
        return sq_fold_ && sq_fold_on_;
    }

private:
    struct Layer {
        int64_t wqkv, wo, wgu, wd, n1, n2;  // base arena offsets (wgu / wd: dense FFN)
        int64_t wr = 0, wex = 0;            // MoE: router [E, d]; experts, each gate, up, down
        // QLoRA: adapter offsets in the trainable arena (A of q, k, v stacked [3r, d]; A of
        // gate, up stacked [2r, d]) and each projection's INT4 bytes / fp16 scales
        int64_t aqkv = 0, bq = 0, bk = 0, bv = 0, ao = 0, bo = 0, agu = 0, bg = 0, bu = 0, ad = 0, bd = 0;
        int64_t pk[7] = {}, sc[7] = {};  // q, k, v, o, gate, up, down
    };
    struct DevScalars;

    bool lora() const { return cfg_.lora_rank > 0; }
    void refresh_low_precision();
    void quantize_base();
    const void* W(int64_t off) const;   // compute-precision trainable weight at arena offset
    const void* WB(int64_t off) const;  // compute-precision base weight at base arena offset
    float* PB(int64_t off) const { return base_dev_ + off; }
    // dequantizes the contiguous projections j0..j1 (q, k, v, o, gate, up, down) of a layer into
    // dst (compute dtype) and returns dst
    const void* dequant_stack(const Layer& ly, int j0, int j1, void* dst, hipStream_t s) const;
    float* P(int64_t off) const { return params_dev_ + off; }
    float* G(int64_t off) const { return grads_dev_ + off; }
    void forward_backward(const int64_t* ids, const int64_t* targets, int64_t B, int64_t S, bool backward,
                          float* loss_out);

    TransformerLMConfig cfg_;
    TrainOptions opt_;
    std::vector<ParamInfo> params_;
    std::vector<ParamInfo> base_;  // QLoRA: the frozen dense model
    int64_t base_arena_ = 0;
    std::vector<Layer> layers_;
    int64_t emb_ = 0, normf_ = 0, head_ = 0;
    int64_t arena_ = 0;
    hipStream_t stream_ = nullptr;
    float* params_dev_ = nullptr;
    float* grads_dev_ = nullptr;
    float* m_dev_ = nullptr;
    float* v_dev_ = nullptr;
    void* low_dev_ = nullptr;  // bf16 shadow weights (AMP)
    float* cos_dev_ = nullptr;
    float* sin_dev_ = nullptr;
    DevScalars* dev_ = nullptr;
    float* one_dev_ = nullptr;
    float* aux_dev_ = nullptr;  // per-layer MoE aux losses [L]
    float* base_dev_ = nullptr;  // frozen base weights (fp32); the trainable arena without QLoRA
    void* base_low_ = nullptr;   // their bf16 shadow (AMP)
    bool q4_fused_ = false;      // QLoRA: base projections dequantized inside the GEMMs
    uint8_t* q4_ = nullptr;      // QLoRA: INT4 projections
    void* q4s_ = nullptr;        //        and their fp16 scales
    std::vector<std::unique_ptr<MoEFFN>> moe_;
    // Step workspace: each buffer of the step (activations kept for the backward, gradients
    // in flight) stays allocated between steps and only grows.  A stream-ordered allocation
    // cannot reuse memory whose free is still queued behind the running step, so fresh
    // per-step allocations would make the host wait for the previous step before enqueueing.
    std::array<DeviceBuffer, 64> ws_;  // fixed size: references to slots stay valid
    DeviceBuffer& workspace(int slot, size_t bytes);
    void* kv_cache_ = nullptr;  // [L][K, V][B][max_seq_len][d] in the compute dtype
    static constexpr int kHistory = 1024;
    aic_step_record* hist_ = nullptr;  // device ring of the last kHistory steps
    int64_t* hist_count_ = nullptr;    // device: records ever written
    int64_t hist_read_ = 0;            // host: records already returned
    float* backup_ = nullptr;          // snapshot: params, m, v (3 arenas) then the device scalars
    int64_t kv_B_ = 0;
    // Gradient-norm partials (fused gradient norm): regions of sq_region_ slots for each layer's
    // weight-gradient launches, one for the LM head's, then the embedding's and the norm weights'
    // sqnorm_k partials; fp64 sums and non-finite flags, zero where no producer writes.  The region
    // size is the largest slot bound (hip::gemm_sq_slots) over the launches that write one.
    int64_t sq_region_ = 0;
    // regions per layer: the grouped launch; with MoE FFNs also the experts' down and gate/up
    // weight gradients and the router's
    int64_t sq_regions_per_layer() const { return cfg_.num_experts > 0 ? 4 : 1; }
    bool sq_fold_ = false;    // the model allows it
    bool sq_fold_on_ = true;  // switched on
    double* sq_part_ = nullptr;  // sq_slots_ partials, then sq_slots_ flags (sq_nf_)
    int* sq_nf_ = nullptr;
    int64_t sq_slots_ = 0;
    double* sq_tmp_ = nullptr;
    int* sq_tmp_nf_ = nullptr;
    Profiler prof_;
};

}  // namespace aic::models
