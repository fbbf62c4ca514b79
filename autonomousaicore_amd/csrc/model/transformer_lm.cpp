#include "transformer_lm.hpp"

#include <algorithm>
#include <array>
#include <initializer_list>
#include <cmath>
#include <cstring>
#include <numeric>
#include <random>
#include <unordered_map>

#include "../kernels/gemm.hpp"
#include "../kernels/kernels.hpp"
#include "../runtime/error.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::models {

// Device-resident scalars of a step, read back with one copy.
struct TransformerLM::DevScalars {
    float loss;
    float scale_used;
    int64_t valid;
    double sqnorm;
    int nonfinite;
    int pad;
    aic_optim_ctl ctl;
    float aux;  // sum of the MoE layers' aux losses of the last forward
    int pad2;
};

namespace {

constexpr int64_t kAlign = 64;  // arena offsets are multiples of 64 elements (256 bytes)

int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// The low-rank term X2 Y2^T a LoRA projection adds to its base product (GemmArgs::X2).
struct LowRank {
    const void* x2;
    int64_t ldx2;
    const void* y2;
    int64_t ldy2, r2, seg_n;
    int y2_kmajor;
};

// A QLoRA base projection (stack) as the GEMM's B operand: packed INT4 values and fp16 group
// scales, dequantized inside the GEMM (packed == nullptr: none; B is the dense operand).
struct Q4B {
    const uint8_t* packed = nullptr;
    const void* scales = nullptr;
    int64_t group = 0;
};

// The rotary embedding of the product's first `cols` columns (the q and k heads; GemmArgs::rope_*).
struct RopeOut {
    const float* cos = nullptr;
    const float* sin = nullptr;
    int64_t cols = 0, hd = 0, seq = 0, start = 0;
};

// SwiGLU of a gate/up product (GemmArgs::glu_*): out = silu(gate) * up, [M, f] with leading dim ld.
struct GluOut {
    void* out = nullptr;
    int64_t f = 0, ld = 0;
};

// SwiGLU's backward fed by the product dh (GemmArgs::dglu_*): gu [M, 2N] in, dgu [M, 2N] out.
struct DGlu {
    const void* gu = nullptr;
    void* out = nullptr;
    int64_t ld = 0;
};

// Sums of squares of an fp32 product for the gradient norm (GemmArgs::sq_*).
struct SqOut {
    double* part = nullptr;
    int* nf = nullptr;
    int64_t cap = 0;
};

void gemm(Profiler& prof, int ta, int tb, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
          const void* B, int64_t ldb, void* C, int64_t ldc, DType ab, DType c, hipStream_t s, const void* R = nullptr,
          int64_t ldr = 0, float beta = 0.0f, float alpha = 1.0f, const LowRank* lr = nullptr, Q4B q4 = {},
          RopeOut rope = {}, GluOut glu = {}, DGlu dglu = {}, SqOut sq = {}) {
    const double es = static_cast<double>(dtype_size(ab)), ec = static_cast<double>(dtype_size(c));
    const double kr = lr ? static_cast<double>(lr->r2) : 0.0;
    // INT4 operand: half a byte per weight plus one fp16 scale per group
    const double bbytes = q4.packed ? 0.5 * N * K + 2.0 * N * K / static_cast<double>(q4.group) : es * N * K;
    auto scope = prof.scope(ta ? kGemmWgrad : (tb ? kGemmFwd : kGemmDgrad), 2.0 * M * N * (K + kr),
                            es * M * K + bbytes + ec * M * N * (R ? 2 : 1), s);
    hip::GemmArgs a;
    a.transA = ta;
    a.transB = tb;
    a.M = M;
    a.N = N;
    a.K = K;
    a.A = A;
    a.lda = lda;
    a.B = B;
    a.ldb = ldb;
    a.C = C;
    a.ldc = ldc;
    a.R = R;
    a.ldr = ldr;
    a.beta = beta;
    a.alpha = alpha;
    a.ab = ab;
    a.c = c;
    if (lr) {
        a.X2 = lr->x2;
        a.ldx2 = lr->ldx2;
        a.Y2 = lr->y2;
        a.ldy2 = lr->ldy2;
        a.r2 = lr->r2;
        a.seg_n = lr->seg_n;
        a.y2_kmajor = lr->y2_kmajor;
    }
    if (q4.packed) {
        a.B = nullptr;
        a.Bq = q4.packed;
        a.Bscale = q4.scales;
        a.scale_t = DType::Float16;
        a.group = q4.group;
    }
    if (rope.cos) {
        a.rope_cos = rope.cos;
        a.rope_sin = rope.sin;
        a.rope_cols = rope.cols;
        a.rope_hd = rope.hd;
        a.rope_seq = rope.seq;
        a.rope_start = rope.start;
    }
    if (glu.out) {
        a.glu_f = glu.f;
        a.glu_out = glu.out;
        a.ld_glu = glu.ld;
    }
    if (dglu.gu) {
        a.dglu_gu = dglu.gu;
        a.dglu_out = dglu.out;
        a.dglu_ld = dglu.ld;
    }
    a.sq_part = sq.part;
    a.sq_nf = sq.nf;
    a.sq_cap = sq.cap;
    hip::gemm(a, s);
}

// Weight gradients dW_i = A_i^T B_i (fp32 out) of independent products in one launch.
void wgrad_grouped(Profiler& prof, std::initializer_list<std::array<const void*, 3>> ops,
                   std::initializer_list<std::array<int64_t, 3>> mnk, DType ab, hipStream_t s, SqOut sq = {}) {
    std::vector<hip::GemmArgs> v;
    double flops = 0.0, bytes = 0.0;
    auto op = ops.begin();
    for (const auto& d : mnk) {
        hip::GemmArgs a;
        a.transA = 1;
        a.transB = 0;
        a.M = d[0];
        a.N = d[1];
        a.K = d[2];
        a.A = (*op)[0];
        a.lda = d[0];
        a.B = (*op)[1];
        a.ldb = d[1];
        a.C = const_cast<void*>((*op)[2]);
        a.ldc = d[1];
        a.ab = ab;
        a.c = DType::Float32;
        v.push_back(a);
        flops += 2.0 * d[0] * d[1] * d[2];
        bytes += static_cast<double>(dtype_size(ab)) * (d[0] * d[2] + d[1] * d[2]) + 4.0 * d[0] * d[1];
        ++op;
    }
    v[0].sq_part = sq.part;  // the whole launch's sums of squares
    v[0].sq_nf = sq.nf;
    v[0].sq_cap = sq.cap;
    auto scope = prof.scope(kGemmWgrad, flops, bytes, s);
    hip::gemm_grouped(v.data(), static_cast<int>(v.size()), s);
}

}  // namespace

// The next token from fp32 logits, as TransformerLM::generate samples it
// (src/models/transformer_lm.cpp:113-206): argmax when temperature <= 0.001 or top_k == 1;
// otherwise softmax(logits / temperature) (sum in double), top-k filtering (std::partial_sort
// by probability) and renormalisation, top-p filtering (std::sort by probability, cumulative
// sum in double, cut at the first index reaching top_p) and renormalisation, then one draw of
// std::discrete_distribution from rng.
int64_t sample_token(const std::vector<float>& l, float temperature, int top_k, float top_p, std::mt19937_64& rng) {
    const int64_t V = static_cast<int64_t>(l.size());
    if (temperature <= 0.001f || top_k == 1) return std::max_element(l.begin(), l.end()) - l.begin();
    std::vector<float> z(l.size());
    float mx = l[0] / temperature;
    for (int64_t v = 0; v < V; ++v) {
        z[v] = l[v] / temperature;
        if (z[v] > mx) mx = z[v];
    }
    std::vector<float> p(l.size());
    double sum = 0.0;
    for (int64_t v = 0; v < V; ++v) {
        p[v] = std::exp(z[v] - mx);
        sum += p[v];
    }
    for (auto& e : p) e /= static_cast<float>(sum);
    if (top_k > 0 && top_k < V) {
        std::vector<int64_t> idx(l.size());
        std::iota(idx.begin(), idx.end(), int64_t{0});
        std::partial_sort(idx.begin(), idx.begin() + top_k, idx.end(), [&p](int64_t a, int64_t b) { return p[a] > p[b]; });
        std::vector<float> kept(l.size(), 0.0f);
        double ks = 0.0;
        for (int i = 0; i < top_k; ++i) {
            kept[idx[i]] = p[idx[i]];
            ks += p[idx[i]];
        }
        for (int i = 0; i < top_k; ++i) kept[idx[i]] /= static_cast<float>(ks);
        p = std::move(kept);
    }
    if (top_p < 1.0f && top_p > 0.0f) {
        std::vector<std::pair<float, int64_t>> pi;
        for (int64_t v = 0; v < V; ++v)
            if (p[v] > 0.0f) pi.push_back({p[v], v});
        std::sort(pi.begin(), pi.end(), [](const auto& a, const auto& b) { return a.first > b.first; });
        double c = 0.0;
        size_t cut = pi.size();
        for (size_t i = 0; i < pi.size(); ++i) {
            c += pi[i].first;
            if (c >= top_p) {
                cut = i + 1;
                break;
            }
        }
        std::vector<float> kept(l.size(), 0.0f);
        double ns = 0.0;
        for (size_t i = 0; i < cut; ++i) {
            kept[pi[i].second] = pi[i].first;
            ns += pi[i].first;
        }
        for (size_t i = 0; i < cut; ++i) kept[pi[i].second] /= static_cast<float>(ns);
        p = std::move(kept);
    }
    std::discrete_distribution<int64_t> dist(p.begin(), p.end());
    return dist(rng);
}

TransformerLM::TransformerLM(const TransformerLMConfig& cfg, const TrainOptions& opt) : cfg_(cfg), opt_(opt) {
    const int64_t V = cfg.vocab_size, d = cfg.hidden_dim, L = cfg.num_layers, H = cfg.num_heads,
                  f = cfg.intermediate_dim;
    AIC_CHECK(V > 0 && d > 0 && L > 0 && H > 0 && f > 0 && cfg.max_seq_len > 0, InvalidArgument,
              "TransformerLM: all sizes must be positive");
    AIC_CHECK(d % H == 0, InvalidArgument, "d_model (", d, ") must be divisible by n_heads (", H, ")");
    AIC_CHECK((d / H) % 2 == 0, InvalidArgument, "head_dim must be even for RoPE");
    AIC_CHECK(cfg.compute == DType::Float32 || cfg.compute == DType::BFloat16, DTypeMismatch,
              "compute dtype must be f32 or bf16");
    const int64_t E = cfg.num_experts;
    AIC_CHECK(E == 0 || (E >= 1 && E <= 64 && cfg.top_k >= 1 && cfg.top_k <= 8 && cfg.top_k <= E), InvalidArgument,
              "MoE: need 1 <= num_experts <= 64 and 1 <= top_k <= min(num_experts, 8)");
    const bool qlora = cfg.lora_rank > 0;
    AIC_CHECK(cfg.lora_rank >= 0 && (!qlora || E == 0), InvalidArgument, "QLoRA: rank >= 0, and not with MoE FFNs");

    // the model's tensors: the trainable arena, or with QLoRA the frozen base arena
    std::vector<ParamInfo>& model = qlora ? base_ : params_;
    int64_t off = 0;
    auto add_to = [](std::vector<ParamInfo>& list, int64_t& o, const std::string& name, std::vector<int64_t> shape) {
        ParamInfo p;
        p.name = name;
        p.shape = shape;
        p.numel = 1;
        for (auto sz : shape) p.numel *= sz;
        p.offset = o;
        o = align_up(o + p.numel);
        list.push_back(p);
        return p.offset;
    };
    auto add = [&](const std::string& name, std::vector<int64_t> shape) { return add_to(model, off, name, shape); };
    emb_ = add("tok_embeddings.weight", {V, d});
    for (int64_t l = 0; l < L; ++l) {
        const std::string pre = "layers." + std::to_string(l) + ".";
        Layer ly;
        // q, k, v are adjacent rows of one [3d, d] matrix; gate, up of one [2f, d] matrix.
        // The alignment padding is zero here because d*d and f*d are multiples of 64 for
        // d % 8 == 0; otherwise the fused GEMMs below are split.
        ly.wqkv = add(pre + "attn.q_proj.weight", {d, d});
        add(pre + "attn.k_proj.weight", {d, d});
        add(pre + "attn.v_proj.weight", {d, d});
        ly.wo = add(pre + "attn.out_proj.weight", {d, d});
        if (E == 0) {
            ly.wgu = add(pre + "ffn.gate_proj.weight", {f, d});
            add(pre + "ffn.up_proj.weight", {f, d});
            ly.wd = add(pre + "ffn.down_proj.weight", {d, f});
        } else {
            // MoETransformerBlock (src/nn/moe.cpp:140-160, 270-280): router Linear(d, E), then
            // expert e's gate [f, d], up [f, d], down [d, f] back to back
            ly.wgu = ly.wd = 0;
            ly.wr = add(pre + "moe.router.gate.weight", {E, d});
            for (int64_t e = 0; e < E; ++e) {
                const std::string ep = pre + "moe.experts." + std::to_string(e) + ".";
                const int64_t g = add(ep + "gate_proj.weight", {f, d});
                if (e == 0) ly.wex = g;
                add(ep + "up_proj.weight", {f, d});
                add(ep + "down_proj.weight", {d, f});
            }
        }
        ly.n1 = add(pre + "norm1.weight", {d});
        ly.n2 = add(pre + "norm2.weight", {d});
        layers_.push_back(ly);
    }
    normf_ = add("norm.weight", {d});
    head_ = cfg.tie_word_embeddings ? emb_ : add("lm_head.weight", {V, d});
    base_arena_ = off;
    arena_ = off;
    int64_t q4_bytes = 0, q4_scales = 0;
    if (qlora) {
        // LoRALinear parameters lora_A / lora_B of the seven projections (src/nn/lora.cpp:31-43)
        const int64_t r = cfg.lora_rank, G = cfg.quant_group;
        AIC_CHECK(G > 0 && G % 2 == 0 && (d * d) % G == 0 && (f * d) % G == 0, InvalidArgument,
                  "QLoRA: the group size must be even and divide d*d and d_ffn*d");
        // A of q, k, v (and of gate, up) must be adjacent to act as one stacked matrix
        AIC_CHECK((r * d) % kAlign == 0 && (r * f) % kAlign == 0, InvalidArgument,
                  "QLoRA: lora_rank * d_model and lora_rank * d_ffn must be multiples of 64");
        int64_t o2 = 0;
        auto lo = [&](const std::string& name, std::vector<int64_t> shape) { return add_to(params_, o2, name, shape); };
        for (int64_t l = 0; l < L; ++l) {
            const std::string pre = "layers." + std::to_string(l) + ".";
            Layer& ly = layers_[static_cast<size_t>(l)];
            ly.aqkv = lo(pre + "attn.q_proj.lora_A", {r, d});
            lo(pre + "attn.k_proj.lora_A", {r, d});
            lo(pre + "attn.v_proj.lora_A", {r, d});
            ly.bq = lo(pre + "attn.q_proj.lora_B", {d, r});
            ly.bk = lo(pre + "attn.k_proj.lora_B", {d, r});
            ly.bv = lo(pre + "attn.v_proj.lora_B", {d, r});
            ly.ao = lo(pre + "attn.out_proj.lora_A", {r, d});
            ly.bo = lo(pre + "attn.out_proj.lora_B", {d, r});
            ly.agu = lo(pre + "ffn.gate_proj.lora_A", {r, d});
            lo(pre + "ffn.up_proj.lora_A", {r, d});
            ly.bg = lo(pre + "ffn.gate_proj.lora_B", {f, r});
            ly.bu = lo(pre + "ffn.up_proj.lora_B", {f, r});
            ly.ad = lo(pre + "ffn.down_proj.lora_A", {r, f});
            ly.bd = lo(pre + "ffn.down_proj.lora_B", {d, r});
            // each stack (q/k/v, o, gate/up, down) contiguous, so that it is one [rows][in] weight
            // whose groups continue across its members; stacks start 256-byte aligned
            const int64_t sizes[7] = {d * d, d * d, d * d, d * d, f * d, f * d, d * f};
            const bool stack_end[7] = {false, false, true, true, false, true, true};
            for (int j = 0; j < 7; ++j) {
                ly.pk[j] = q4_bytes;
                q4_bytes += sizes[j] / 2;
                ly.sc[j] = q4_scales;
                q4_scales += sizes[j] / G;
                if (stack_end[j]) {
                    q4_bytes = (q4_bytes + 255) / 256 * 256;
                    q4_scales = (q4_scales + 127) / 128 * 128;
                }
            }
        }
        arena_ = o2;
        // bf16 base projections dequantized inside the GEMM kernels (which need these multiples);
        // otherwise each projection stack is dequantized into a scratch buffer before its GEMM
        q4_fused_ = cfg.compute == DType::BFloat16 && G % 64 == 0 && d % 64 == 0 && f % 64 == 0;
    }
    AIC_CHECK((d * d) % kAlign == 0 && (f * d) % kAlign == 0, InvalidArgument,
              "d_model*d_model and d_ffn*d_model must be multiples of 64 (fused q/k/v and gate/up projections)");

    AIC_HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    const size_t bytes = sizeof(float) * static_cast<size_t>(arena_);
    AIC_HIP_CHECK(hipMalloc(&params_dev_, bytes));
    AIC_HIP_CHECK(hipMalloc(&grads_dev_, bytes));
    AIC_HIP_CHECK(hipMalloc(&m_dev_, bytes));
    AIC_HIP_CHECK(hipMalloc(&v_dev_, bytes));
    AIC_HIP_CHECK(hipMemsetAsync(params_dev_, 0, bytes, stream_));
    AIC_HIP_CHECK(hipMemsetAsync(grads_dev_, 0, bytes, stream_));
    AIC_HIP_CHECK(hipMemsetAsync(m_dev_, 0, bytes, stream_));
    AIC_HIP_CHECK(hipMemsetAsync(v_dev_, 0, bytes, stream_));
    AIC_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&hist_), sizeof(aic_step_record) * kHistory));
    AIC_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&hist_count_), sizeof(int64_t)));
    AIC_HIP_CHECK(hipMemsetAsync(hist_count_, 0, sizeof(int64_t), stream_));
    if (cfg.compute == DType::BFloat16) {
        AIC_HIP_CHECK(hipMalloc(&low_dev_, sizeof(uint16_t) * static_cast<size_t>(arena_)));
        AIC_HIP_CHECK(hipMemsetAsync(low_dev_, 0, sizeof(uint16_t) * static_cast<size_t>(arena_), stream_));
    }
    if (qlora) {
        AIC_HIP_CHECK(hipMalloc(&base_dev_, sizeof(float) * static_cast<size_t>(base_arena_)));
        AIC_HIP_CHECK(hipMemsetAsync(base_dev_, 0, sizeof(float) * static_cast<size_t>(base_arena_), stream_));
        if (cfg.compute == DType::BFloat16) {
            AIC_HIP_CHECK(hipMalloc(&base_low_, sizeof(uint16_t) * static_cast<size_t>(base_arena_)));
            AIC_HIP_CHECK(hipMemsetAsync(base_low_, 0, sizeof(uint16_t) * static_cast<size_t>(base_arena_), stream_));
        }
        AIC_HIP_CHECK(hipMalloc(&q4_, static_cast<size_t>(q4_bytes)));
        AIC_HIP_CHECK(hipMalloc(&q4s_, sizeof(uint16_t) * static_cast<size_t>(q4_scales)));
        AIC_HIP_CHECK(hipMemsetAsync(q4_, 0, static_cast<size_t>(q4_bytes), stream_));
        AIC_HIP_CHECK(hipMemsetAsync(q4s_, 0, sizeof(uint16_t) * static_cast<size_t>(q4_scales), stream_));
    } else {
        base_dev_ = params_dev_;
        base_low_ = low_dev_;
    }

    const int64_t hd = d / H, half = hd / 2;
    std::vector<float> c(static_cast<size_t>(cfg.max_seq_len * half)), s(c.size());
    hip::rope_tables_host(c.data(), s.data(), cfg.max_seq_len, hd, cfg.rope_theta);
    AIC_HIP_CHECK(hipMalloc(&cos_dev_, sizeof(float) * c.size()));
    AIC_HIP_CHECK(hipMalloc(&sin_dev_, sizeof(float) * s.size()));
    AIC_HIP_CHECK(hipMemcpy(cos_dev_, c.data(), sizeof(float) * c.size(), hipMemcpyHostToDevice));
    AIC_HIP_CHECK(hipMemcpy(sin_dev_, s.data(), sizeof(float) * s.size(), hipMemcpyHostToDevice));

    DevScalars init{};
    init.ctl.scale = opt.use_loss_scaler ? opt.scaler.initial_scale : 1.0f;
    init.ctl.use_scaler = opt.use_loss_scaler ? 1 : 0;
    init.ctl.growth_factor = opt.scaler.growth_factor;
    init.ctl.backoff_factor = opt.scaler.backoff_factor;
    init.ctl.growth_interval = opt.scaler.growth_interval;
    init.ctl.min_scale = opt.scaler.min_scale;
    init.ctl.max_scale = opt.scaler.max_scale;
    init.ctl.max_grad_norm = opt.max_grad_norm;
    init.scale_used = init.ctl.scale;
    AIC_HIP_CHECK(hipMalloc(&dev_, sizeof(DevScalars)));
    AIC_HIP_CHECK(hipMemcpy(dev_, &init, sizeof(DevScalars), hipMemcpyHostToDevice));
    const float one = 1.0f;
    AIC_HIP_CHECK(hipMalloc(&one_dev_, sizeof(float)));
    AIC_HIP_CHECK(hipMemcpy(one_dev_, &one, sizeof(float), hipMemcpyHostToDevice));
    // fused gradient norm: models with an untied head, whose every gradient comes from the
    // layers' weight-gradient GEMMs (the grouped launch; with MoE FFNs also the experts' and the
    // router's), the head's GEMM, the embedding backward and the norm weights (checked against
    // the tensor list)
    if (!qlora && !cfg.tie_word_embeddings) {
        const int64_t ffn = E > 0 ? E * d + E * 3 * f * d : 3 * f * d;
        int64_t covered = L * (4 * d * d + ffn + 2 * d) + 2 * V * d + d, listed = 0;
        for (const ParamInfo& p : params_) listed += p.numel;
        sq_fold_ = covered == listed;
    }
    if (sq_fold_) {
        // one region size for all producers: the largest of their slot bounds
        auto prod = [](int64_t M, int64_t N) {
            hip::GemmArgs a;
            a.M = M;
            a.N = N;
            return a;
        };
        const hip::GemmArgs head = prod(V, d);
        sq_region_ = hip::gemm_sq_slots(&head, 1);
        if (E > 0) {
            const hip::GemmArgs attn[2] = {prod(3 * d, d), prod(d, d)};
            const hip::GemmArgs router = prod(E, d);
            sq_region_ = std::max({sq_region_, hip::gemm_sq_slots(attn, 2), hip::gemm_sq_slots(&router, 1),
                                   hip::gemm_ragged_sq_slots(d, f, static_cast<int>(E)),
                                   hip::gemm_ragged_sq_slots(2 * f, d, static_cast<int>(E))});
        } else {
            const hip::GemmArgs layer[4] = {prod(3 * d, d), prod(d, d), prod(2 * f, d), prod(d, f)};
            sq_region_ = std::max(sq_region_, hip::gemm_sq_slots(layer, 4));
        }
        std::vector<int64_t> sizes(1, V * d);
        sizes.resize(2 * L + 2, d);
        sq_slots_ = (L * sq_regions_per_layer() + 1) * sq_region_ +
                    hip::sqnorm_slots(sizes.data(), static_cast<int>(sizes.size()));
        const int64_t nt = hip::sqnorm_reduce_tmp(sq_slots_);
        // the partials, then the flags, in one allocation (cleared by one fill per step)
        AIC_HIP_CHECK(hipMalloc(&sq_part_, (sizeof(double) + sizeof(int)) * static_cast<size_t>(sq_slots_)));
        sq_nf_ = reinterpret_cast<int*>(sq_part_ + sq_slots_);
        AIC_HIP_CHECK(hipMalloc(&sq_tmp_, sizeof(double) * static_cast<size_t>(nt)));
        AIC_HIP_CHECK(hipMalloc(&sq_tmp_nf_, sizeof(int) * static_cast<size_t>(nt)));
    }
    if (E > 0) {
        AIC_HIP_CHECK(hipMalloc(&aux_dev_, sizeof(float) * static_cast<size_t>(L)));
        AIC_HIP_CHECK(hipMemset(aux_dev_, 0, sizeof(float) * static_cast<size_t>(L)));
        for (int64_t l = 0; l < L; ++l) {
            moe_.push_back(std::make_unique<MoEFFN>(d, f, E, cfg.top_k, cfg.aux_loss_coef, cfg.compute));
            moe_.back()->set_profiler(&prof_);
        }
    }
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
}

TransformerLM::~TransformerLM() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    moe_.clear();  // their buffers are freed on stream_, so before it is destroyed
    for (auto& b : ws_) b.reset();
    if (kv_cache_ && stream_) {
        (void)hipFreeAsync(kv_cache_, stream_);
        (void)hipStreamSynchronize(stream_);
    }
    for (void* p : {static_cast<void*>(params_dev_), static_cast<void*>(grads_dev_), static_cast<void*>(m_dev_),
                    static_cast<void*>(v_dev_), low_dev_, static_cast<void*>(cos_dev_), static_cast<void*>(sin_dev_),
                    static_cast<void*>(dev_), static_cast<void*>(one_dev_), static_cast<void*>(aux_dev_)})
        if (p) (void)hipFree(p);
    for (void* p : {static_cast<void*>(hist_), static_cast<void*>(hist_count_), static_cast<void*>(backup_),
                    static_cast<void*>(sq_part_), static_cast<void*>(sq_tmp_), static_cast<void*>(sq_tmp_nf_)})
        if (p) (void)hipFree(p);
    if (lora())
        for (void* p : {static_cast<void*>(base_dev_), base_low_, static_cast<void*>(q4_), q4s_})
            if (p) (void)hipFree(p);
    if (stream_) {
        try {
            stream_scratch_release(stream_);
        } catch (...) {  // a destructor does not throw
        }
        (void)hipStreamSynchronize(stream_);
        (void)hipStreamDestroy(stream_);
    }
}

int64_t TransformerLM::num_params() const {
    int64_t n = 0;
    for (const auto& p : params_) n += p.numel;
    return n;
}

void TransformerLM::refresh_low_precision() {
    if (low_dev_) hip::cast_f32_bf16(params_dev_, low_dev_, arena_, stream_);
    if (lora() && base_low_) hip::cast_f32_bf16(base_dev_, base_low_, base_arena_, stream_);
}

const void* TransformerLM::W(int64_t off) const {
    if (low_dev_) return static_cast<const uint16_t*>(low_dev_) + off;
    return params_dev_ + off;
}

const void* TransformerLM::WB(int64_t off) const {
    if (base_low_) return static_cast<const uint16_t*>(base_low_) + off;
    return base_dev_ + off;
}

namespace {
// base-arena offset and element count of projection j (q, k, v, o, gate, up, down)
void proj_of(int64_t wqkv, int64_t wo, int64_t wgu, int64_t wd, int64_t d, int64_t f, int j, int64_t& off, int64_t& n) {
    const int64_t offs[7] = {wqkv, wqkv + d * d, wqkv + 2 * d * d, wo, wgu, wgu + f * d, wd};
    const int64_t ns[7] = {d * d, d * d, d * d, d * d, f * d, f * d, d * f};
    off = offs[j];
    n = ns[j];
}
}  // namespace

void TransformerLM::quantize_base() {
    const int64_t d = cfg_.hidden_dim, f = cfg_.intermediate_dim;
    for (const Layer& ly : layers_)
        for (int j = 0; j < 7; ++j) {
            int64_t off, n;
            proj_of(ly.wqkv, ly.wo, ly.wgu, ly.wd, d, f, j, off, n);
            hip::int4_quantize(base_dev_ + off, n, cfg_.quant_group, q4_ + ly.pk[j],
                               static_cast<uint16_t*>(q4s_) + ly.sc[j], DType::Float16, stream_);
        }
}

const void* TransformerLM::dequant_stack(const Layer& ly, int j0, int j1, void* dst, hipStream_t s) const {
    // a stack's projections are contiguous (bytes and scales), one weight of the summed size
    const int64_t d = cfg_.hidden_dim, f = cfg_.intermediate_dim;
    int64_t n = 0;
    for (int j = j0; j <= j1; ++j) {
        int64_t off, nj;
        proj_of(ly.wqkv, ly.wo, ly.wgu, ly.wd, d, f, j, off, nj);
        n += nj;
    }
    hip::int4_dequant(q4_ + ly.pk[j0], static_cast<const uint16_t*>(q4s_) + ly.sc[j0], DType::Float16, n,
                      cfg_.quant_group, dst, cfg_.compute, s);
    return dst;
}

namespace {
// host holds the tensors back to back in list order, without the alignment padding
void scatter_to_device(const float* host, const std::vector<ParamInfo>& ps, int64_t arena, float* dev, hipStream_t s) {
    std::vector<float> full(static_cast<size_t>(arena), 0.0f);
    int64_t src = 0;
    for (const auto& p : ps) {
        std::memcpy(full.data() + p.offset, host + src, sizeof(float) * static_cast<size_t>(p.numel));
        src += p.numel;
    }
    AIC_HIP_CHECK(hipMemcpyAsync(dev, full.data(), sizeof(float) * full.size(), hipMemcpyHostToDevice, s));
    AIC_HIP_CHECK(hipStreamSynchronize(s));
}
}  // namespace

void TransformerLM::set_params(const float* host) {
    scatter_to_device(host, params_, arena_, params_dev_, stream_);
    refresh_low_precision();
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
}

void TransformerLM::set_base_params(const float* host) {
    AIC_CHECK(lora(), InvalidState, "set_base_params: the model has no frozen base (lora_rank == 0); use set_params");
    scatter_to_device(host, base_, base_arena_, base_dev_, stream_);
    quantize_base();
    refresh_low_precision();
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
}

namespace {
void gather_host(const float* dev, const std::vector<ParamInfo>& ps, int64_t arena, float* host, hipStream_t s) {
    std::vector<float> full(static_cast<size_t>(arena));
    AIC_HIP_CHECK(hipMemcpyAsync(full.data(), dev, sizeof(float) * full.size(), hipMemcpyDeviceToHost, s));
    AIC_HIP_CHECK(hipStreamSynchronize(s));
    int64_t dst = 0;
    for (const auto& p : ps) {
        std::memcpy(host + dst, full.data() + p.offset, sizeof(float) * static_cast<size_t>(p.numel));
        dst += p.numel;
    }
}
}  // namespace

void TransformerLM::get_params(float* host) const { gather_host(params_dev_, params_, arena_, host, stream_); }
void TransformerLM::get_base_params(float* host) const {
    AIC_CHECK(lora(), InvalidState, "get_base_params: the model has no frozen base (lora_rank == 0); use get_params");
    gather_host(base_dev_, base_, base_arena_, host, stream_);
}
void TransformerLM::get_grads(float* host) const { gather_host(grads_dev_, params_, arena_, host, stream_); }

int64_t TransformerLM::moe_routing(int64_t layer, int64_t* host, int64_t cap) const {
    AIC_CHECK(!moe_.empty(), InvalidArgument, "moe_routing: not a MoE model");
    AIC_CHECK(layer >= 0 && layer < static_cast<int64_t>(moe_.size()), OutOfRange, "moe_routing: layer ", layer,
              " of ", moe_.size());
    const MoEFFN& m = *moe_[static_cast<size_t>(layer)];
    const int64_t n = m.tokens() * m.top_k();
    AIC_CHECK(n > 0, InvalidArgument, "moe_routing: no forward has run");
    AIC_CHECK(host && cap >= n, OutOfRange, "moe_routing: ", n, " values, room for ", cap);
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
    AIC_HIP_CHECK(hipMemcpy(host, m.idx(), sizeof(int64_t) * static_cast<size_t>(n), hipMemcpyDeviceToHost));
    return m.tokens();
}

void TransformerLM::get_adam_state(float* m, float* v, int64_t* step) const {
    if (m) gather_host(m_dev_, params_, arena_, m, stream_);
    if (v) gather_host(v_dev_, params_, arena_, v, stream_);
    if (step) {
        DevScalars h{};
        AIC_HIP_CHECK(hipMemcpyAsync(&h, dev_, sizeof(h), hipMemcpyDeviceToHost, stream_));
        AIC_HIP_CHECK(hipStreamSynchronize(stream_));
        *step = h.ctl.step;
    }
}

namespace {
std::vector<float> gather_packed(const float* dev, const std::vector<ParamInfo>& ps, int64_t arena, hipStream_t s) {
    int64_t n = 0;
    for (const auto& p : ps) n += p.numel;
    std::vector<float> out(static_cast<size_t>(n));
    gather_host(dev, ps, arena, out.data(), s);
    return out;
}
}  // namespace

void TransformerLM::save_checkpoint(const std::string& path, const CheckpointMeta& meta, bool with_optimizer) {
    struct Src {
        const ParamInfo* p;
        const float* host;
    };
    std::vector<float> tp = gather_packed(params_dev_, params_, arena_, stream_);
    std::vector<float> bp;
    std::vector<Src> model;
    int64_t o = 0;
    for (const auto& p : params_) {
        model.push_back({&p, tp.data() + o});
        o += p.numel;
    }
    if (lora()) {
        bp = gather_packed(base_dev_, base_, base_arena_, stream_);
        o = 0;
        for (const auto& p : base_) {
            model.push_back({&p, bp.data() + o});
            o += p.numel;
        }
    }
    std::vector<std::string> names;
    for (const auto& m : model) names.push_back(m.p->name);
    std::vector<CheckpointTensorRef> refs;
    for (size_t i : module_order(names)) {
        const ParamInfo& p = *model[i].p;
        refs.push_back({p.name, p.shape, 0, model[i].host, sizeof(float) * static_cast<uint64_t>(p.numel)});
    }
    std::vector<float> m, v;
    int64_t step = 0, good = 0;
    float scale = 1.0f;
    if (with_optimizer) {
        m = gather_packed(m_dev_, params_, arena_, stream_);
        v = gather_packed(v_dev_, params_, arena_, stream_);
        DevScalars h{};
        AIC_HIP_CHECK(hipMemcpyAsync(&h, dev_, sizeof(h), hipMemcpyDeviceToHost, stream_));
        AIC_HIP_CHECK(hipStreamSynchronize(stream_));
        step = h.ctl.step;
        good = h.ctl.good_steps;
        scale = h.ctl.scale;
        std::vector<std::string> tn;
        for (const auto& p : params_) tn.push_back(p.name);
        const std::vector<size_t> order = module_order(tn);
        std::vector<int64_t> offs(params_.size());
        o = 0;
        for (size_t i = 0; i < params_.size(); ++i) {
            offs[i] = o;
            o += params_[i].numel;
        }
        for (int which = 0; which < 2; ++which)
            for (size_t i : order) {
                const ParamInfo& p = params_[i];
                refs.push_back({std::string(which ? "optimizer.exp_avg_sq." : "optimizer.exp_avg.") + p.name, p.shape,
                                0, (which ? v.data() : m.data()) + offs[i],
                                sizeof(float) * static_cast<uint64_t>(p.numel)});
            }
        refs.push_back({"optimizer.step", {1}, 4, &step, sizeof(int64_t)});
        refs.push_back({"amp.loss_scale", {1}, 0, &scale, sizeof(float)});
        refs.push_back({"amp.good_steps", {1}, 4, &good, sizeof(int64_t)});
    }
    write_checkpoint(path, meta, refs);
}

CheckpointMeta TransformerLM::load_checkpoint(const std::string& path, bool* has_optimizer) {
    CheckpointMeta meta;
    std::vector<CheckpointTensor> ts;
    read_checkpoint(path, meta, ts);
    struct Dst {
        const ParamInfo* p;
        int64_t packed;  // offset in the packed host copy
        int arena;       // 0 trainable, 1 base
    };
    std::unordered_map<std::string, Dst> where;
    int64_t o = 0;
    for (const auto& p : params_) {
        where[p.name] = {&p, o, 0};
        o += p.numel;
    }
    if (lora()) {
        o = 0;
        for (const auto& p : base_) {
            where[p.name] = {&p, o, 1};
            o += p.numel;
        }
    }
    std::vector<float> tp = gather_packed(params_dev_, params_, arena_, stream_);
    std::vector<float> bp = lora() ? gather_packed(base_dev_, base_, base_arena_, stream_) : std::vector<float>();
    std::vector<float> m, v;
    bool got_t = false, got_b = false, got_m = false, got_v = false, got_ctl = false;
    int64_t step = -1, good = -1;
    float scale = -1.0f;
    auto check_f32 = [&](const CheckpointTensor& t, const ParamInfo& p) {
        AIC_CHECK(t.dims == p.shape, ShapeMismatch, "Shape mismatch loading tensor '", t.name, "'");
        AIC_CHECK(t.dtype == 0 && t.data.size() == sizeof(float) * static_cast<size_t>(p.numel), DTypeMismatch,
                  "DType mismatch loading tensor '", t.name, "'");
    };
    for (const auto& t : ts) {
        const std::string kM = "optimizer.exp_avg.", kV = "optimizer.exp_avg_sq.";
        if (auto it = where.find(t.name); it != where.end()) {
            check_f32(t, *it->second.p);
            float* dst = (it->second.arena ? bp.data() : tp.data()) + it->second.packed;
            std::memcpy(dst, t.data.data(), t.data.size());
            (it->second.arena ? got_b : got_t) = true;
        } else if (t.name.rfind(kV, 0) == 0 || t.name.rfind(kM, 0) == 0) {
            const bool is_v = t.name.rfind(kV, 0) == 0;
            auto jt = where.find(t.name.substr(is_v ? kV.size() : kM.size()));
            if (jt == where.end() || jt->second.arena != 0) continue;
            check_f32(t, *jt->second.p);
            std::vector<float>& dst = is_v ? v : m;
            if (dst.empty()) dst = gather_packed(is_v ? v_dev_ : m_dev_, params_, arena_, stream_);
            std::memcpy(dst.data() + jt->second.packed, t.data.data(), t.data.size());
            (is_v ? got_v : got_m) = true;
        } else if (t.name == "optimizer.step" && t.dtype == 4 && t.data.size() == 8) {
            std::memcpy(&step, t.data.data(), 8);
            got_ctl = true;
        } else if (t.name == "amp.good_steps" && t.dtype == 4 && t.data.size() == 8) {
            std::memcpy(&good, t.data.data(), 8);
            got_ctl = true;
        } else if (t.name == "amp.loss_scale" && t.dtype == 0 && t.data.size() == 4) {
            std::memcpy(&scale, t.data.data(), 4);
            got_ctl = true;
        }
    }
    if (got_t) scatter_to_device(tp.data(), params_, arena_, params_dev_, stream_);
    if (got_b) {
        scatter_to_device(bp.data(), base_, base_arena_, base_dev_, stream_);
        quantize_base();
    }
    if (got_m) scatter_to_device(m.data(), params_, arena_, m_dev_, stream_);
    if (got_v) scatter_to_device(v.data(), params_, arena_, v_dev_, stream_);
    if (got_ctl) {
        DevScalars h{};
        AIC_HIP_CHECK(hipMemcpyAsync(&h, dev_, sizeof(h), hipMemcpyDeviceToHost, stream_));
        AIC_HIP_CHECK(hipStreamSynchronize(stream_));
        if (step >= 0) h.ctl.step = static_cast<int>(step);
        if (good >= 0) h.ctl.good_steps = static_cast<int>(good);
        if (scale > 0.0f) h.ctl.scale = scale;
        AIC_HIP_CHECK(hipMemcpyAsync(dev_, &h, sizeof(h), hipMemcpyHostToDevice, stream_));
    }
    refresh_low_precision();
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
    if (has_optimizer) *has_optimizer = got_m && got_v && step >= 0;
    return meta;
}

void TransformerLM::init_normal(uint64_t seed, float std, bool residual_scaling) {
    const float rs = residual_scaling ? 1.0f / std::sqrt(2.0f * static_cast<float>(cfg_.num_layers)) : 1.0f;
    uint64_t off = 0;
    for (const auto& p : base_params()) {
        const bool is_norm = p.shape.size() == 1;
        if (is_norm) {
            hip::fill_const(base_dev_ + p.offset, p.numel, 1.0f, stream_);
        } else {
            const bool resid = p.name.find("out_proj") != std::string::npos ||
                               p.name.find("down_proj") != std::string::npos;
            hip::fill_normal(base_dev_ + p.offset, p.numel, seed, off, 0.0f, std * (resid ? rs : 1.0f), stream_);
        }
        off += static_cast<uint64_t>(p.numel);
    }
    if (lora()) {
        // the QLoRA configuration: A ~ N(0, std), B = 0, so the adapted model starts as the base
        quantize_base();
        for (const auto& p : params_) {
            if (p.name.find("lora_B") != std::string::npos) hip::fill_const(params_dev_ + p.offset, p.numel, 0.0f, stream_);
            else hip::fill_normal(params_dev_ + p.offset, p.numel, seed, off, 0.0f, std, stream_);
            off += static_cast<uint64_t>(p.numel);
        }
    }
    refresh_low_precision();
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
}

DeviceBuffer& TransformerLM::workspace(int slot, size_t bytes) {
    AIC_CHECK(slot >= 0 && static_cast<size_t>(slot) < ws_.size(), InvalidState, "workspace slot ", slot);
    DeviceBuffer& b = ws_[static_cast<size_t>(slot)];
    if (b.bytes() < bytes) b = DeviceBuffer(bytes, stream_);  // the old one is freed in stream order
    return b;
}

void TransformerLM::forward_backward(const int64_t* ids, const int64_t* targets, int64_t B, int64_t S, bool backward,
                                     float* loss_out) {
    AIC_CHECK(B > 0 && S > 0, InvalidArgument, "batch and sequence must be positive");
    AIC_CHECK(S <= cfg_.max_seq_len, OutOfRange, "sequence length ", S, " exceeds max_seq_len ", cfg_.max_seq_len);
    const hipStream_t s = stream_;
    const DType dt = cfg_.compute;
    const size_t es = dtype_size(dt);
    const int64_t T = B * S, d = cfg_.hidden_dim, f = cfg_.intermediate_dim, V = cfg_.vocab_size,
                  H = cfg_.num_heads, hd = d / H, L = cfg_.num_layers;
    const float eps = cfg_.rms_norm_eps;
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    // causal attention: S(S+1)/2 (query, key) pairs per head, 2 products of 2*hd FLOPs each
    const double attn_flops = 2.0 * static_cast<double>(B * H) * static_cast<double>(S) * (S + 1) * hd;

    int slot = 0;  // workspace slots in a fixed order
    auto act = [&](int64_t elems) -> DeviceBuffer& { return workspace(slot++, es * static_cast<size_t>(elems)); };
    auto f32 = [&](int64_t elems) -> DeviceBuffer& {
        return workspace(slot++, sizeof(float) * static_cast<size_t>(elems));
    };

    // ---- activations kept for the backward ----
    DeviceBuffer& xs = act((L + 1) * T * d);  // residual stream x_0 .. x_L
    const bool moe = cfg_.num_experts > 0;
    DeviceBuffer &h1 = act(L * T * d), &qkv = act(L * T * 3 * d), &ob = act(L * T * d), &x1 = act(L * T * d),
                 &h2 = act(L * T * d), &gu = act(moe ? 0 : L * T * 2 * f), &am = act(moe ? 0 : L * T * f);
    DeviceBuffer &r1 = f32(L * T), &r2 = f32(L * T), &lse = f32(L * T * H);
    DeviceBuffer &hf = act(T * d), &rf = f32(T), &logits = act(T * V), &lse_ce = f32(T);
    // QLoRA: each layer's adapter inputs x A^T (q/k/v stacked [T,3r], o [T,r], gate/up [T,2r],
    // down [T,r]) kept for the backward.  The frozen INT4 base stays INT4 in HBM: with bf16
    // operands the GEMMs dequantize it in their operand load (q4f); otherwise one projection
    // stack at a time is dequantized into a scratch buffer right before each GEMM that reads it,
    // in the forward and again in the backward.
    const bool ql = lora();
    const bool q4f = ql && q4_fused_ && T >= 8;
    const int64_t r = cfg_.lora_rank;
    const float lsc = ql ? cfg_.lora_alpha / static_cast<float>(r) : 0.0f;
    DeviceBuffer& xa_all = act(ql ? L * T * 7 * r : 0);
    DeviceBuffer& wbuf = act(ql && !q4f ? std::max(3 * d * d, 2 * f * d) : 0);
    auto at = [&](const DeviceBuffer& b, int64_t elem) {
        return static_cast<void*>(static_cast<char*>(b.get()) + es * static_cast<size_t>(elem));
    };
    auto atf = [&](const DeviceBuffer& b, int64_t elem) { return b.as<float>() + elem; };
    auto xaq = [&](int64_t l) { return at(xa_all, l * T * 7 * r); };
    auto xao = [&](int64_t l) { return at(xa_all, l * T * 7 * r + T * 3 * r); };
    auto xagu = [&](int64_t l) { return at(xa_all, l * T * 7 * r + T * 4 * r); };
    auto xad = [&](int64_t l) { return at(xa_all, l * T * 7 * r + T * 6 * r); };
    // a projection stack's base weight (projections j0..j1 of q, k, v, o, gate, up, down): the
    // arena, or with QLoRA (QuantizedLinear::forward, src/nn/quantization.cpp:669-679) the INT4
    // stack as an in-GEMM operand (wq) or dequantized into wbuf (wbase)
    auto wbase = [&](const Layer& ly, int64_t off, int j0, int j1) -> const void* {
        if (!ql) return WB(off);
        if (q4f) return nullptr;
        return dequant_stack(ly, j0, j1, wbuf.get(), s);
    };
    auto wq = [&](const Layer& ly, int j0) -> Q4B {
        return q4f ? Q4B{q4_ + ly.pk[j0], static_cast<const uint16_t*>(q4s_) + ly.sc[j0], cfg_.quant_group} : Q4B{};
    };
    // the frozen model's gradients are not formed with QLoRA
    auto GB = [&](int64_t off) -> float* { return ql ? nullptr : G(off); };
    // LoRA's rank-r products (LoRALinear, src/nn/lora.cpp:75-93) in one pass over the large
    // operand where the kernel takes the shape (bf16, widths % 256), else as GEMMs
    auto lora_pass = [&](const hip::LoraSkinny& q, double flops) {
        if (dt != DType::BFloat16 || !hip::lora_skinny_ok(q)) return false;
        const double big = es * static_cast<double>(q.T) * q.N;  // the operand the pass streams
        const double small = es * static_cast<double>(q.T) * (q.N / q.n_seg) * q.r_seg;
        auto _p = prof_.scope(kLora, flops, big + (q.out1 ? small : 0.0) + (q.Z ? small : 0.0), s);
        hip::lora_skinny(q, s);
        return true;
    };
    // xs = s x A^T, A [R, in] (the adapters' A of a projection stack, stacked)
    auto lora_xa = [&](const void* x, int64_t in, int64_t a_off, int64_t R, void* out) {
        hip::LoraSkinny q;
        q.Y = x;
        q.ldy = in;
        q.T = T;
        q.N = in;
        q.n_seg = in;
        q.r_seg = R;
        q.W = W(a_off);
        q.w_n = 1;
        q.w_j = in;
        q.out1 = out;
        q.ldo1 = R;
        q.scale = lsc;
        if (!lora_pass(q, 2.0 * T * in * R))
            gemm(prof_, 0, 1, T, R, in, x, in, W(a_off), in, out, R, dt, dt, s, nullptr, 0, 0.0f, lsc);
    };

    // ---- forward (TransformerLM::forward, src/models/transformer_lm.cpp:50-62) ----
    {
        auto _p = prof_.scope(kEmbedFwd, 0.0, 2.0 * es * T * d + 8.0 * T, s);
        hip::embed_fwd(ids, T, WB(emb_), V, d, at(xs, 0), dt, s);
    }
    for (int64_t l = 0; l < L; ++l) {
        const Layer& ly = layers_[l];
        void* x = at(xs, l * T * d);
        void* xn = at(xs, (l + 1) * T * d);
        void* h1l = at(h1, l * T * d);
        void* qkvl = at(qkv, l * T * 3 * d);
        void* ol = at(ob, l * T * d);
        void* x1l = at(x1, l * T * d);
        void* h2l = at(h2, l * T * d);
        void* gul = moe ? nullptr : at(gu, l * T * 2 * f);
        void* aml = moe ? nullptr : at(am, l * T * f);
        {
            auto _p = prof_.scope(kNormFwd, 0.0, 2.0 * es * T * d + 4.0 * T, s);
            hip::rmsnorm_fwd(x, d, PB(ly.n1), h1l, d, atf(r1, l * T), T, d, eps, dt, s);
        }
        // LoRA (LoRALinear::forward, src/nn/lora.cpp:75-93): xs = s (x A^T) is formed first (A of
        // q, k, v stacked, [3r, d]); the base GEMM then adds xs B^T to its accumulators, each
        // output column block (q, k, v) with its own r columns of xs and its own B
        LowRank lq{};
        if (ql) {
            lora_xa(h1l, d, ly.aqkv, 3 * r, xaq(l));
            lq = LowRank{xaq(l), 3 * r, W(ly.bq), r, r, d, 0};
        }
        // q and k leave the projection rotated (RotaryPositionEmbedding::forward in the GEMM's
        // epilogue where its shape allows, else a rope pass right after it)
        gemm(prof_, 0, 1, T, 3 * d, d, h1l, d, wbase(ly, ly.wqkv, 0, 2), d, qkvl, 3 * d, dt, dt, s, nullptr, 0, 0.0f,
             1.0f, ql ? &lq : nullptr, wq(ly, 0), RopeOut{cos_dev_, sin_dev_, 2 * d, hd, S, 0});
        {
            auto _p = prof_.scope(kAttnFwd, attn_flops, 4.0 * es * T * d, s);
            hip::attn_fwd(qkvl, static_cast<char*>(qkvl) + es * d, static_cast<char*>(qkvl) + es * 2 * d, 3 * d, ol,
                          d, atf(lse, l * T * H), B, H, S, hd, true, scale, dt, s);
        }
        LowRank lo_{};
        if (ql) {
            lora_xa(ol, d, ly.ao, r, xao(l));
            lo_ = LowRank{xao(l), r, W(ly.bo), r, r, 0, 0};
        }
        gemm(prof_, 0, 1, T, d, d, ol, d, wbase(ly, ly.wo, 3, 3), d, x1l, d, dt, dt, s, x, d, 0.0f, 1.0f,
             ql ? &lo_ : nullptr, wq(ly, 3));
        {
            auto _p = prof_.scope(kNormFwd, 0.0, 2.0 * es * T * d + 4.0 * T, s);
            hip::rmsnorm_fwd(x1l, d, PB(ly.n2), h2l, d, atf(r2, l * T), T, d, eps, dt, s);
        }
        if (moe) {
            // MoELayer::forward (src/nn/moe.cpp:155-253) with the residual x1 added by the combine
            moe_[l]->forward(h2l, T, W(ly.wr), W(ly.wex), x1l, xn, aux_dev_ + l, s);
            continue;
        }
        LowRank lg{};
        if (ql) {
            lora_xa(h2l, d, ly.agu, 2 * r, xagu(l));
            lg = LowRank{xagu(l), 2 * r, W(ly.bg), r, r, f, 0};
        }
        // gate/up, with SwiGLU's silu(gate) * up written by the GEMM's epilogue where its shape
        // allows (else a swiglu pass right after it)
        gemm(prof_, 0, 1, T, 2 * f, d, h2l, d, wbase(ly, ly.wgu, 4, 5), d, gul, 2 * f, dt, dt, s, nullptr, 0, 0.0f,
             1.0f, ql ? &lg : nullptr, wq(ly, 4), RopeOut{}, GluOut{aml, f, f});
        LowRank ld_{};
        if (ql) {
            lora_xa(aml, f, ly.ad, r, xad(l));
            ld_ = LowRank{xad(l), r, W(ly.bd), r, r, 0, 0};
        }
        gemm(prof_, 0, 1, T, d, f, aml, f, wbase(ly, ly.wd, 6, 6), f, xn, d, dt, dt, s, x1l, d, 0.0f, 1.0f,
             ql ? &ld_ : nullptr, wq(ly, 6));
    }
    void* xL = at(xs, L * T * d);
    {
        auto _p = prof_.scope(kNormFwd, 0.0, 2.0 * es * T * d + 4.0 * T, s);
        hip::rmsnorm_fwd(xL, d, PB(normf_), hf.get(), d, rf.as<float>(), T, d, eps, dt, s);
    }
    gemm(prof_, 0, 1, T, V, d, hf.get(), d, WB(head_), d, logits.get(), V, dt, dt, s);

    // ---- loss (cross_entropy mean, ignore_index -100, src/loss/cross_entropy.cpp:149-290) ----
    // A training step fuses the loss's backward into its forward: the logits are read once and
    // overwritten by their gradient (scaled by the loss scaler's current scale).
    const float* gscale = opt_.use_loss_scaler ? &dev_->ctl.scale : one_dev_;
    if (backward) {
        AIC_HIP_CHECK(hipMemcpyAsync(&dev_->scale_used, &dev_->ctl.scale, sizeof(float), hipMemcpyDeviceToDevice, s));
        auto _p = prof_.scope(kCeFwdBwd, 0.0, 2.0 * es * T * V + 28.0 * T, s);
        hip::ce_fwd_bwd(logits.get(), V, targets, T, V, -100, nullptr, lse_ce.as<float>(), &dev_->loss, &dev_->valid,
                        gscale, dt, s);
    } else {
        auto _p = prof_.scope(kCeFwd, 0.0, es * T * V + 16.0 * T, s);
        hip::ce_fwd(logits.get(), V, targets, T, V, -100, nullptr, lse_ce.as<float>(), &dev_->loss, &dev_->valid, dt,
                    s);
    }
    // total_loss = cross_entropy + total_aux_loss (tests/unit/test_moe.cpp:224-228)
    if (moe) hip::moe_aux_total(aux_dev_, L, &dev_->loss, &dev_->aux, s);
    if (!backward) {
        if (loss_out) {
            AIC_HIP_CHECK(hipMemcpyAsync(loss_out, &dev_->loss, sizeof(float), hipMemcpyDeviceToHost, s));
            AIC_HIP_CHECK(hipStreamSynchronize(s));
        }
        return;
    }

    // ---- backward (autograd::backward, src/autograd/engine.cpp:116-189, as a fixed schedule) ----
    void* dl = logits.get();
    // dx: the residual-stream gradient at a layer's output; dxm: at its attention block's output
    // (the FFN's RMSNorm backward writes it next to dx, which the dense model's deferred
    // down-projection weight gradient still reads)
    DeviceBuffer &dx = act(T * d), &dxm = act(T * d), &dh = act(T * d), &dqkv = act(T * 3 * d),
                 &dgu = act(moe ? 0 : T * 2 * f), &da = act(moe ? 0 : T * f), &dxa = act(ql ? T * 3 * r : 0);
    // LoRA backward of one projection (LoRALinear, src/nn/lora.cpp:75-93, through autograd):
    // with y += xs B^T and xs = s (x A^T) kept from the forward,
    //   dB = dy^T xs, dxa = s dy B   (then dA = dxa^T x, and dx += dxa A in the base dgrad GEMM)
    auto lora_b_bwd = [&](const void* dy, int64_t lddy, int64_t n_out, const void* xs, int64_t ldxs, int64_t boff,
                          void* dxa_out, int64_t lddxa) {
        gemm(prof_, 1, 0, n_out, r, T, dy, lddy, xs, ldxs, G(boff), r, dt, DType::Float32, s);
        gemm(prof_, 0, 0, T, r, n_out, dy, lddy, W(boff), r, dxa_out, lddxa, dt, dt, s, nullptr, 0, 0.0f, lsc);
    };
    // The same for a stack of nb projections whose outputs are the n_out-column blocks of dy
    // [T, nb n_out] and whose B's are stacked in the arena (boffs[j] = boffs[0] + j n_out r):
    // dB and dxa of all of them from one pass over dy
    auto lora_bwd = [&](const void* dy, int64_t n_out, int nb, const void* xs, const int64_t* boffs, void* dxa_out) {
        bool stacked = true;
        for (int j = 1; j < nb; ++j) stacked = stacked && boffs[j] == boffs[0] + j * n_out * r;
        hip::LoraSkinny q;
        q.Y = dy;
        q.ldy = nb * n_out;
        q.T = T;
        q.N = nb * n_out;
        q.n_seg = n_out;
        q.r_seg = r;
        q.W = W(boffs[0]);
        q.w_n = r;
        q.w_j = 1;
        q.out1 = dxa_out;
        q.ldo1 = nb * r;
        q.scale = lsc;
        q.Z = xs;
        q.ldz = nb * r;
        q.out2 = G(boffs[0]);
        q.o2n = r;
        q.o2j = 1;
        if (stacked && lora_pass(q, 4.0 * T * nb * n_out * r)) return;
        for (int j = 0; j < nb; ++j)
            lora_b_bwd(static_cast<const char*>(dy) + es * j * n_out, nb * n_out, n_out,
                       static_cast<const char*>(xs) + es * j * r, nb * r, boffs[j],
                       static_cast<char*>(dxa_out) + es * j * r, nb * r);
    };
    // dA = dxa^T x for A [R, in] (stacked A's of a projection stack)
    auto lora_da = [&](const void* x, int64_t in, const void* dxa_in, int64_t R, int64_t a_off) {
        hip::LoraSkinny q;
        q.Y = x;
        q.ldy = in;
        q.T = T;
        q.N = in;
        q.n_seg = in;
        q.r_seg = R;
        q.Z = dxa_in;
        q.ldz = R;
        q.out2 = G(a_off);
        q.o2n = 1;
        q.o2j = in;
        if (!lora_pass(q, 2.0 * T * in * R))
            gemm(prof_, 1, 0, R, in, T, dxa_in, R, x, in, G(a_off), in, dt, DType::Float32, s);
    };
    // the gradient norm's partial sums, where the step forms it from the producers (sq_fold)
    const bool fold = sq_fold_ && sq_fold_on_;
    const int64_t RPL = sq_regions_per_layer();
    auto sq_region = [&](int64_t r) {
        return fold ? SqOut{sq_part_ + r * sq_region_, sq_nf_ + r * sq_region_, sq_region_} : SqOut{};
    };
    auto slots = [&](int64_t r) { return SqSlots{sq_part_ + r * sq_region_, sq_nf_ + r * sq_region_, sq_region_}; };
    // every slot starts at zero: a launch writes only the slots of its path, which can change with
    // the token count (T not a multiple of 64 leaves the tile kernels)
    if (fold) {
        auto _p = prof_.scope(kGradNorm, 0.0, 12.0 * sq_slots_, s);
        hip::sqnorm_clear(sq_part_, sq_nf_, sq_slots_, s);
    }
    if (!ql)
        gemm(prof_, 1, 0, V, d, T, dl, V, hf.get(), d, G(head_), d, dt, DType::Float32, s, nullptr, 0, 0.0f, 1.0f,
             nullptr, {}, RopeOut{}, GluOut{}, DGlu{}, sq_region(L * RPL));
    gemm(prof_, 0, 0, T, d, V, dl, V, WB(head_), d, dh.get(), d, dt, dt, s);
    // The norms' weight gradients: each backward leaves its partial rows in dwp and one launch
    // after the layer loop reduces them all (the same sums in the same order), where the shape
    // allows; the optimizer tail is their only reader.
    const bool defer_dw = !ql && d % 8 == 0;
    const int64_t prow = hip::rmsnorm_bwd_part_rows(T);
    float* dwp = defer_dw ? f32((2 * L + 1) * prow * d).as<float>() : nullptr;
    std::vector<const float*> dw_parts;
    std::vector<float*> dw_dst;
    auto norm_bwd = [&](const void* dy, const void* xn, const float* w, const float* rms, const void* dres,
                        void* out, float* dwt) {
        if (defer_dw && dwt) {
            float* part = dwp + static_cast<int64_t>(dw_parts.size()) * prow * d;
            hip::rmsnorm_bwd_deferred(dy, d, xn, d, w, rms, dres, d, out, d, part, T, d, dt, s);
            dw_parts.push_back(part);
            dw_dst.push_back(dwt);
        } else {
            hip::rmsnorm_bwd(dy, d, xn, d, w, rms, dres, d, out, d, dwt, false, T, d, dt, s);
        }
    };
    {
        auto _p = prof_.scope(kNormBwd, 0.0, 3.0 * es * T * d + 4.0 * T, s);
        norm_bwd(dh.get(), xL, PB(normf_), rf.as<float>(), nullptr, dx.get(), GB(normf_));
    }
    for (int64_t l = L - 1; l >= 0; --l) {
        const Layer& ly = layers_[l];
        void* x = at(xs, l * T * d);
        void* h1l = at(h1, l * T * d);
        void* qkvl = at(qkv, l * T * 3 * d);
        void* ol = at(ob, l * T * d);
        void* x1l = at(x1, l * T * d);
        void* h2l = at(h2, l * T * d);
        if (moe) {
            // x_{l+1} = x1 + moe(h2); d total_loss / d aux_l = 1 (times the loss scale)
            const SqSlots msq[3] = {slots(l * RPL + 1), slots(l * RPL + 2), slots(l * RPL + 3)};
            moe_[l]->backward(dx.get(), 1.0f, dh.get(), G(ly.wr), G(ly.wex), s, gscale, fold ? msq : nullptr);
        } else {
            void* gul = at(gu, l * T * 2 * f);
            void* aml = at(am, l * T * f);
            // x_{l+1} = x1 + down(silu(gate(h2)) * up(h2))
            LowRank ld_{};
            if (ql) {
                lora_bwd(dx.get(), d, 1, xad(l), &ly.bd, dxa.get());
                lora_da(aml, f, dxa.get(), r, ly.ad);
                ld_ = LowRank{dxa.get(), r, W(ly.ad), f, r, 0, 1};
            }  // else: the down-projection weight gradient joins the layer's grouped launch below
            // da = dx W_d goes straight into SwiGLU's backward in the GEMM's epilogue (dgu from da
            // and the saved gate/up) where its shape allows, else through da and a swiglu pass
            gemm(prof_, 0, 0, T, f, d, dx.get(), d, wbase(ly, ly.wd, 6, 6), f, da.get(), f, dt, dt, s, nullptr, 0,
                 0.0f, 1.0f, ql ? &ld_ : nullptr, wq(ly, 6), RopeOut{}, GluOut{}, DGlu{gul, dgu.get(), 2 * f});
            LowRank lg{};
            if (ql) {
                const int64_t bs[2] = {ly.bg, ly.bu};
                lora_bwd(dgu.get(), f, 2, xagu(l), bs, dxa.get());
                lora_da(h2l, d, dxa.get(), 2 * r, ly.agu);
                lg = LowRank{dxa.get(), 2 * r, W(ly.agu), d, 2 * r, 0, 1};
            }  // else: the gate/up weight gradient joins the layer's grouped launch below (dgu is
               // not written again before it)
            gemm(prof_, 0, 0, T, d, 2 * f, dgu.get(), 2 * f, wbase(ly, ly.wgu, 4, 5), d, dh.get(), d, dt, dt, s,
                 nullptr, 0, 0.0f, 1.0f, ql ? &lg : nullptr, wq(ly, 4));
        }
        {
            auto _p = prof_.scope(kNormBwd, 0.0, 4.0 * es * T * d + 4.0 * T, s);
            norm_bwd(dh.get(), x1l, PB(ly.n2), atf(r2, l * T), dx.get(), dxm.get(), GB(ly.n2));
        }
        // x1 = x + out_proj(attn(rope(q), rope(k), v))
        LowRank lo_{};
        if (ql) {
            lora_bwd(dxm.get(), d, 1, xao(l), &ly.bo, dxa.get());
            lora_da(ol, d, dxa.get(), r, ly.ao);
            lo_ = LowRank{dxa.get(), r, W(ly.ao), d, r, 0, 1};
        }  // else: the out_proj weight gradient joins the layer's grouped launch below
        gemm(prof_, 0, 0, T, d, d, dxm.get(), d, wbase(ly, ly.wo, 3, 3), d, dh.get(), d, dt, dt, s, nullptr, 0, 0.0f,
             1.0f, ql ? &lo_ : nullptr, wq(ly, 3));
        {
            // counted as dP, dV, dK, dQ (twice the forward); the recomputed S = Q K^T is not.  The
            // rotary embedding's backward (RoPEBackward) leaves the kernels with dq and dk.
            auto _p = prof_.scope(kAttnBwd, 2.0 * attn_flops, 8.0 * es * T * d, s);
            hip::attn_bwd(qkvl, static_cast<char*>(qkvl) + es * d, static_cast<char*>(qkvl) + es * 2 * d, 3 * d, ol,
                          dh.get(), d, atf(lse, l * T * H), dqkv.get(), static_cast<char*>(dqkv.get()) + es * d,
                          static_cast<char*>(dqkv.get()) + es * 2 * d, 3 * d, B, H, S, hd, true, scale, dt, s,
                          cos_dev_, sin_dev_);
        }
        LowRank lq{};
        if (ql) {
            const int64_t bs[3] = {ly.bq, ly.bk, ly.bv};
            lora_bwd(dqkv.get(), d, 3, xaq(l), bs, dxa.get());
            lora_da(h1l, d, dxa.get(), 3 * r, ly.aqkv);
            lq = LowRank{dxa.get(), 3 * r, W(ly.aqkv), d, 3 * r, 0, 1};
        } else if (moe) {
            // dWqkv = dqkv^T h1 and dWo = dxm^T o in one launch
            wgrad_grouped(prof_, {{dqkv.get(), h1l, G(ly.wqkv)}, {dxm.get(), ol, G(ly.wo)}},
                          {{3 * d, d, T}, {d, d, T}}, dt, s, sq_region(l * RPL));
        } else {
            // the layer's four weight gradients in one launch: dWqkv = dqkv^T h1, dWo = dxm^T o,
            // dWgu = dgu^T h2 and dWd = dx^T am (at the 1B shape 192 + 64 + 352 + 176 tiles of
            // 256x256: a little over three full rounds of the chip instead of four partial ones)
            wgrad_grouped(prof_,
                          {{dqkv.get(), h1l, G(ly.wqkv)}, {dxm.get(), ol, G(ly.wo)},
                           {dgu.get(), at(h2, l * T * d), G(ly.wgu)}, {dx.get(), at(am, l * T * f), G(ly.wd)}},
                          {{3 * d, d, T}, {d, d, T}, {2 * f, d, T}, {d, f, T}}, dt, s, sq_region(l * RPL));
        }
        gemm(prof_, 0, 0, T, d, 3 * d, dqkv.get(), 3 * d, wbase(ly, ly.wqkv, 0, 2), d, dh.get(), d, dt, dt, s, nullptr,
             0, 0.0f, 1.0f, ql ? &lq : nullptr, wq(ly, 0));
        {
            auto _p = prof_.scope(kNormBwd, 0.0, 4.0 * es * T * d + 4.0 * T, s);
            norm_bwd(dh.get(), x, PB(ly.n1), atf(r1, l * T), dxm.get(), dx.get(), GB(ly.n1));
        }
    }
    if (!dw_parts.empty()) {
        const double n = static_cast<double>(dw_parts.size());
        auto _p = prof_.scope(kNormBwd, 0.0, 4.0 * n * prow * d + 4.0 * n * d, s);
        hip::rmsnorm_dw_reduce(dw_parts.data(), dw_dst.data(), static_cast<int>(dw_parts.size()), T, d, s);
    }
    if (!ql) {
        auto _p = prof_.scope(kEmbedBwd, 0.0, es * T * d + 4.0 * V * d + 8.0 * T, s);
        hip::embed_bwd(ids, T, dx.get(), V, d, G(emb_), cfg_.tie_word_embeddings, dt, s);
    }

    // ---- optimizer tail: scaler -> clip_grad_norm_ -> AdamW (src/train/trainer.cpp:70-95) ----
    const float* gp[1] = {grads_dev_};
    const int64_t sizes[1] = {arena_};
    if (fold) {
        // the weight gradients' partial sums came from their GEMMs; the embedding's and the
        // norm weights' are added here, then every slot in a fixed order
        std::vector<const float*> eg(1, G(emb_));
        std::vector<int64_t> en(1, V * d);
        for (const Layer& ly : layers_) {
            eg.push_back(G(ly.n1));
            eg.push_back(G(ly.n2));
        }
        eg.push_back(G(normf_));
        en.resize(eg.size(), d);
        auto _p = prof_.scope(kGradNorm, 0.0, 4.0 * (V * d + (2 * L + 1) * d) + 12.0 * sq_slots_, s);
        const int64_t pass0 = (L * RPL + 1) * sq_region_;
        hip::sqnorm_partials(eg.data(), en.data(), static_cast<int>(eg.size()), sq_part_ + pass0, sq_nf_ + pass0, s);
        hip::sqnorm_reduce(sq_part_, sq_nf_, sq_slots_, sq_tmp_, sq_tmp_nf_, &dev_->sqnorm, &dev_->nonfinite, s);
        hip::optim_finalize(&dev_->sqnorm, &dev_->nonfinite, &dev_->ctl, s);
    } else {
        auto _p = prof_.scope(kGradNorm, 0.0, 4.0 * arena_, s);
        hip::grad_sqnorm_multi(gp, sizes, 1, &dev_->sqnorm, &dev_->nonfinite, s);
        hip::optim_finalize(&dev_->sqnorm, &dev_->nonfinite, &dev_->ctl, s);
    }
    float* pp[1] = {params_dev_};
    float* mp[1] = {m_dev_};
    float* vp[1] = {v_dev_};
    void* lp[1] = {low_dev_};
    const auto& a = opt_.adamw;
    {
        auto _p = prof_.scope(kAdamW, 0.0, (28.0 + (low_dev_ ? 2.0 : 0.0)) * arena_, s);
        hip::adamw_multi(pp, gp, mp, vp, low_dev_ ? lp : nullptr, sizes, 1, a.lr, a.beta1, a.beta2, a.eps,
                         a.weight_decay, 0, &dev_->ctl, s);
    }
    hip::step_record(&dev_->loss, moe ? &dev_->aux : nullptr, &dev_->ctl, &dev_->scale_used, hist_, hist_count_,
                     kHistory, s);
}

int TransformerLM::step_history(aic_step_record* out, int cap, int64_t* dropped) {
    if (dropped) *dropped = 0;
    if (cap <= 0) return 0;
    int64_t total = 0;
    std::vector<aic_step_record> ring(kHistory);
    AIC_HIP_CHECK(hipMemcpyAsync(&total, hist_count_, sizeof(int64_t), hipMemcpyDeviceToHost, stream_));
    AIC_HIP_CHECK(hipMemcpyAsync(ring.data(), hist_, sizeof(aic_step_record) * kHistory, hipMemcpyDeviceToHost,
                                 stream_));
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
    int64_t first = std::max(hist_read_, total - kHistory);
    if (dropped) *dropped = first - hist_read_;
    const int64_t n = std::min<int64_t>(total - first, cap);
    for (int64_t i = 0; i < n; ++i) out[i] = ring[static_cast<size_t>((first + i) % kHistory)];
    hist_read_ = first + n;
    return static_cast<int>(n);
}

void TransformerLM::snapshot() {
    const size_t a = sizeof(float) * static_cast<size_t>(arena_);
    if (!backup_) AIC_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&backup_), 3 * a + sizeof(DevScalars)));
    char* b = reinterpret_cast<char*>(backup_);
    AIC_HIP_CHECK(hipMemcpyAsync(b, params_dev_, a, hipMemcpyDeviceToDevice, stream_));
    AIC_HIP_CHECK(hipMemcpyAsync(b + a, m_dev_, a, hipMemcpyDeviceToDevice, stream_));
    AIC_HIP_CHECK(hipMemcpyAsync(b + 2 * a, v_dev_, a, hipMemcpyDeviceToDevice, stream_));
    AIC_HIP_CHECK(hipMemcpyAsync(b + 3 * a, dev_, sizeof(DevScalars), hipMemcpyDeviceToDevice, stream_));
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
}

void TransformerLM::restore() {
    AIC_CHECK(backup_, InvalidState, "restore: no snapshot taken");
    const size_t a = sizeof(float) * static_cast<size_t>(arena_);
    const char* b = reinterpret_cast<const char*>(backup_);
    AIC_HIP_CHECK(hipMemcpyAsync(params_dev_, b, a, hipMemcpyDeviceToDevice, stream_));
    AIC_HIP_CHECK(hipMemcpyAsync(m_dev_, b + a, a, hipMemcpyDeviceToDevice, stream_));
    AIC_HIP_CHECK(hipMemcpyAsync(v_dev_, b + 2 * a, a, hipMemcpyDeviceToDevice, stream_));
    AIC_HIP_CHECK(hipMemcpyAsync(dev_, b + 3 * a, sizeof(DevScalars), hipMemcpyDeviceToDevice, stream_));
    refresh_low_precision();
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
}

void TransformerLM::forward_step(const int64_t* ids, int64_t B, int64_t S, int64_t start_pos, float* logits) {
    const int64_t V = cfg_.vocab_size, d = cfg_.hidden_dim, L = cfg_.num_layers, H = cfg_.num_heads,
                  f = cfg_.intermediate_dim, hd = d / H, T = B * S, MS = cfg_.max_seq_len;
    AIC_CHECK(ids && logits && B > 0 && S > 0 && start_pos >= 0, InvalidArgument, "forward_step: bad arguments");
    AIC_CHECK(start_pos + S <= MS, OutOfRange, "forward_step: positions up to ", start_pos + S,
              " exceed max_seq_len ", MS);
    AIC_CHECK(start_pos == 0 || B == kv_B_, InvalidState,
              "forward_step: a continuation (start_pos > 0) must keep the batch size of its sequence");
    const DType dt = cfg_.compute;
    const size_t es = dtype_size(dt);
    const float eps = cfg_.rms_norm_eps, scale = 1.0f / std::sqrt(static_cast<float>(hd));
    hipStream_t s = stream_;
    if (start_pos == 0 && B != kv_B_) {
        if (kv_cache_) AIC_HIP_CHECK(hipFreeAsync(kv_cache_, s));
        kv_cache_ = nullptr;
        AIC_HIP_CHECK(hipMallocAsync(&kv_cache_, es * static_cast<size_t>(L * 2 * B * MS * d), s));
        kv_B_ = B;
    }
    int slot = 40;  // the decode path's own workspace slots (its sizes differ from the step's)
    auto act = [&](int64_t elems) -> DeviceBuffer& { return workspace(slot++, es * static_cast<size_t>(elems)); };
    auto f32 = [&](int64_t elems) -> DeviceBuffer& {
        return workspace(slot++, sizeof(float) * static_cast<size_t>(elems));
    };
    auto at = [&](const DeviceBuffer& b, int64_t elem) {
        return static_cast<void*>(static_cast<char*>(b.get()) + es * static_cast<size_t>(elem));
    };
    const bool moe = cfg_.num_experts > 0, ql = lora();
    const int64_t r = cfg_.lora_rank;
    const float lsc = ql ? cfg_.lora_alpha / static_cast<float>(r) : 0.0f;
    DeviceBuffer &xa = act(T * d), &xb = act(T * d), &h = act(T * d), &qkv = act(T * 3 * d), &ob = act(T * d),
                 &x1 = act(T * d), &gu = act(moe ? 0 : T * 2 * f), &am = act(moe ? 0 : T * f), &rr = f32(T),
                 &lse = f32(start_pos == 0 ? T * H : 0), &xs = act(ql ? T * 7 * r : 0);
    // QLoRA base projections as in the training step: in-GEMM INT4 operands, or dequantized
    // stack by stack into a scratch buffer (fp32 operands, or fewer than 8 rows)
    const bool q4f = ql && q4_fused_ && T >= 8;
    DeviceBuffer& wbuf = act(ql && !q4f ? std::max(3 * d * d, 2 * f * d) : 0);
    auto wbase = [&](const Layer& ly, int64_t off, int j0, int j1) -> const void* {
        if (!ql) return WB(off);
        if (q4f) return nullptr;
        return dequant_stack(ly, j0, j1, wbuf.get(), s);
    };
    auto wq = [&](const Layer& ly, int j0) -> Q4B {
        return q4f ? Q4B{q4_ + ly.pk[j0], static_cast<const uint16_t*>(q4s_) + ly.sc[j0], cfg_.quant_group} : Q4B{};
    };
    hip::embed_fwd(ids, T, WB(emb_), V, d, xa.get(), dt, s);
    void* x = xa.get();
    void* xn = xb.get();
    for (int64_t l = 0; l < L; ++l) {
        const Layer& ly = layers_[l];
        hip::rmsnorm_fwd(x, d, PB(ly.n1), h.get(), d, rr.as<float>(), T, d, eps, dt, s);
        LowRank lq{};
        if (ql) {
            gemm(prof_, 0, 1, T, 3 * r, d, h.get(), d, W(ly.aqkv), d, xs.get(), 3 * r, dt, dt, s, nullptr, 0, 0.0f, lsc);
            lq = LowRank{xs.get(), 3 * r, W(ly.bq), r, r, d, 0};
        }
        gemm(prof_, 0, 1, T, 3 * d, d, h.get(), d, wbase(ly, ly.wqkv, 0, 2), d, qkv.get(), 3 * d, dt, dt, s, nullptr,
             0, 0.0f, 1.0f, ql ? &lq : nullptr, wq(ly, 0));
        hip::rope(qkv.get(), 3 * d, B, S, 2 * H, hd, start_pos, cos_dev_, sin_dev_, false, dt, s);
        // the new keys and values join the cache at rows start_pos .. start_pos + S - 1
        char* kc = static_cast<char*>(kv_cache_) + es * static_cast<size_t>(l * 2 * B * MS * d);
        char* vc = kc + es * static_cast<size_t>(B * MS * d);
        for (int64_t b = 0; b < B; ++b)
            for (int kv = 0; kv < 2; ++kv)
                AIC_HIP_CHECK(hipMemcpy2DAsync((kv ? vc : kc) + es * static_cast<size_t>((b * MS + start_pos) * d),
                                               es * d, static_cast<char*>(qkv.get()) + es * ((b * S) * 3 * d + (1 + kv) * d),
                                               es * 3 * d, es * d, S, hipMemcpyDeviceToDevice, s));
        if (start_pos == 0)  // a fresh sequence: the flash kernel on the new rows is the same causal attention
            hip::attn_fwd(qkv.get(), static_cast<char*>(qkv.get()) + es * d, static_cast<char*>(qkv.get()) + es * 2 * d,
                          3 * d, ob.get(), d, lse.as<float>(), B, H, S, hd, true, scale, dt, s);
        else
            hip::attn_cached(qkv.get(), 3 * d, kc, vc, d, MS, ob.get(), d, B, H, S, start_pos, hd, scale, dt, s);
        LowRank lo_{};
        if (ql) {
            gemm(prof_, 0, 1, T, r, d, ob.get(), d, W(ly.ao), d, xs.get(), r, dt, dt, s, nullptr, 0, 0.0f, lsc);
            lo_ = LowRank{xs.get(), r, W(ly.bo), r, r, 0, 0};
        }
        gemm(prof_, 0, 1, T, d, d, ob.get(), d, wbase(ly, ly.wo, 3, 3), d, x1.get(), d, dt, dt, s, x, d, 0.0f, 1.0f,
             ql ? &lo_ : nullptr, wq(ly, 3));
        hip::rmsnorm_fwd(x1.get(), d, PB(ly.n2), h.get(), d, rr.as<float>(), T, d, eps, dt, s);
        if (moe) {
            moe_[l]->forward(h.get(), T, W(ly.wr), W(ly.wex), x1.get(), xn, aux_dev_ + l, s);
        } else {
            LowRank lg{};
            if (ql) {
                gemm(prof_, 0, 1, T, 2 * r, d, h.get(), d, W(ly.agu), d, xs.get(), 2 * r, dt, dt, s, nullptr, 0, 0.0f,
                     lsc);
                lg = LowRank{xs.get(), 2 * r, W(ly.bg), r, r, f, 0};
            }
            gemm(prof_, 0, 1, T, 2 * f, d, h.get(), d, wbase(ly, ly.wgu, 4, 5), d, gu.get(), 2 * f, dt, dt, s,
                 nullptr, 0, 0.0f, 1.0f, ql ? &lg : nullptr, wq(ly, 4));
            hip::swiglu_fwd(gu.get(), at(gu, f), 2 * f, am.get(), f, T, f, dt, s);
            LowRank ld_{};
            if (ql) {
                gemm(prof_, 0, 1, T, r, f, am.get(), f, W(ly.ad), f, xs.get(), r, dt, dt, s, nullptr, 0, 0.0f, lsc);
                ld_ = LowRank{xs.get(), r, W(ly.bd), r, r, 0, 0};
            }
            gemm(prof_, 0, 1, T, d, f, am.get(), f, wbase(ly, ly.wd, 6, 6), f, xn, d, dt, dt, s, x1.get(), d, 0.0f,
                 1.0f, ql ? &ld_ : nullptr, wq(ly, 6));
        }
        std::swap(x, xn);
    }
    hip::rmsnorm_fwd(x, d, PB(normf_), h.get(), d, rr.as<float>(), T, d, eps, dt, s);
    gemm(prof_, 0, 1, T, V, d, h.get(), d, WB(head_), d, logits, V, dt, DType::Float32, s);
}

std::vector<int64_t> TransformerLM::generate(const std::vector<int64_t>& prompt, int64_t max_new_tokens,
                                             float temperature, int top_k, float top_p, int64_t eos_token_id,
                                             uint64_t seed) {
    AIC_CHECK(max_new_tokens >= 0, InvalidArgument, "max_new_tokens must be non-negative");
    const int64_t V = cfg_.vocab_size;
    std::vector<int64_t> out = prompt.empty() ? std::vector<int64_t>{0} : prompt;
    const int64_t n0 = static_cast<int64_t>(out.size());
    AIC_CHECK(n0 + max_new_tokens <= cfg_.max_seq_len + 1, OutOfRange, "generate: ", n0, " + ", max_new_tokens,
              " tokens exceed max_seq_len ", cfg_.max_seq_len);
    for (int64_t t : out) AIC_CHECK(t >= 0 && t < V, OutOfRange, "generate: token ", t, " outside the vocabulary");
    std::mt19937_64 rng(seed);
    DeviceBuffer ids(sizeof(int64_t) * static_cast<size_t>(n0), stream_), logits(sizeof(float) * n0 * V, stream_);
    AIC_HIP_CHECK(hipMemcpyAsync(ids.get(), out.data(), sizeof(int64_t) * n0, hipMemcpyHostToDevice, stream_));
    forward_step(ids.as<int64_t>(), 1, n0, 0, logits.as<float>());  // the prompt in one prefill
    std::vector<float> l(static_cast<size_t>(V));
    AIC_HIP_CHECK(hipMemcpyAsync(l.data(), logits.as<float>() + (n0 - 1) * V, sizeof(float) * V, hipMemcpyDeviceToHost,
                                 stream_));
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
    for (int64_t step = 0; step < max_new_tokens; ++step) {
        const int64_t next = sample_token(l, temperature, top_k, top_p, rng);
        out.push_back(next);
        if ((eos_token_id >= 0 && next == eos_token_id) || step + 1 == max_new_tokens) break;
        AIC_HIP_CHECK(hipMemcpyAsync(ids.get(), &next, sizeof(int64_t), hipMemcpyHostToDevice, stream_));
        forward_step(ids.as<int64_t>(), 1, 1, n0 + step, logits.as<float>());
        AIC_HIP_CHECK(hipMemcpyAsync(l.data(), logits.get(), sizeof(float) * V, hipMemcpyDeviceToHost, stream_));
        AIC_HIP_CHECK(hipStreamSynchronize(stream_));
    }
    return out;
}

void TransformerLM::train_step(const int64_t* ids, const int64_t* targets, int64_t B, int64_t S) {
    forward_backward(ids, targets, B, S, true, nullptr);
}

float TransformerLM::eval_loss(const int64_t* ids, const int64_t* targets, int64_t B, int64_t S) {
    float loss = 0.0f;
    forward_backward(ids, targets, B, S, false, &loss);
    return loss;
}

StepStats TransformerLM::last_stats() {
    DevScalars h{};
    AIC_HIP_CHECK(hipMemcpyAsync(&h, dev_, sizeof(h), hipMemcpyDeviceToHost, stream_));
    AIC_HIP_CHECK(hipStreamSynchronize(stream_));
    StepStats st;
    st.loss = h.loss;
    st.aux_loss = cfg_.num_experts > 0 ? h.aux : 0.0f;
    st.grad_norm = h.ctl.grad_norm;
    st.found_inf = h.ctl.skip != 0;
    st.loss_scale = h.scale_used;
    st.step = h.ctl.step;
    return st;
}

void TransformerLM::synchronize() { AIC_HIP_CHECK(hipStreamSynchronize(stream_)); }

}  // namespace aic::models
