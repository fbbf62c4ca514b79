// Step telemetry and anomaly detection behind the interface of the reference's
// TelemetryTracker (include/autonomous/telemetry.hpp; behaviour of
// src/autonomous/telemetry.cpp:126-275).  Rules, per recorded step:
//   * loss EMAs (short and long alpha) and a gradient-norm EMA (short alpha), each seeded by the
//     first finite value it sees, non-finite values skipped;
//   * the population variance of the finite losses among the last `window` steps;
//   * TFLOP/s = 6 * parameters * tokens/s (tokens/s from total tokens / seconds when not given);
//   * host memory from /proc/meminfo, GPU memory from hipMemGetInfo;
//   * the anomaly, first match: non-finite loss, non-finite gradient norm, divergence (the last 3
//     losses each above 1.4x the long EMA of their step), gradient explosion (at least 5 steps,
//     norm above 4x its EMA, or above 100 while the EMA is ~0), vanishing gradient (at least 5
//     steps, norm below 1e-7), GPU memory under 8% free.
// The statistics it consumes come from the device-side step history of TransformerLM, read in
// batches, so the training loop needs no host synchronisation per step.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>
#include <string>

namespace aic {

enum class AnomalyType : int {
    None = 0,
    NanOrInfLoss,
    NanOrInfGradient,
    LossDivergence,
    GradientExplosion,
    GradientVanishing,
    MemoryCritical
};
const char* anomaly_name(AnomalyType t);

struct HardwareMemoryStats {
    uint64_t host_total = 0, host_free = 0, gpu_total = 0, gpu_free = 0;
};

struct TelemetrySnapshot {
    int64_t step = 0;
    float loss = 0.0f, loss_ema_short = 0.0f, loss_ema_long = 0.0f, loss_variance = 0.0f;
    float grad_norm = 0.0f, grad_norm_ema = 0.0f, lr = 0.0f, tokens_per_sec = 0.0f, estimated_tflops = 0.0f;
    HardwareMemoryStats memory;
    AnomalyType anomaly = AnomalyType::None;
    std::string to_json() const;
};

class TelemetryTracker {
public:
    explicit TelemetryTracker(size_t window = 50, float alpha_short = 0.8f, float alpha_long = 0.98f);
    // device_index < 0: no GPU memory query
    TelemetrySnapshot record_step(int64_t step, float loss, float grad_norm, float lr, float tokens_per_sec,
                                  double step_seconds, int64_t total_tokens, int64_t model_params, int device_index);
    static HardwareMemoryStats query_memory(int device_index);
    bool is_nan_or_inf() const;
    bool is_diverging(float threshold_ratio = 1.4f, int min_consecutive = 3) const;
    bool is_gradient_exploding(float spike_factor = 4.0f) const;
    bool is_gradient_vanishing(float min_norm = 1e-7f) const;
    bool is_memory_critical(float min_free_ratio = 0.08f) const;
    size_t count() const { return size_; }
    const TelemetrySnapshot& latest() const { return latest_; }
    void reset();

private:
    struct Ema {
        float alpha;
        float value = 0.0f;
        bool seeded = false;
        void add(float x);
    };
    struct Record {
        float loss, grad_norm, loss_ema_long;
    };
    const Record& from_newest(size_t i) const;  // i = 0: the latest step
    float window_loss_variance() const;
    static float tflops(int64_t model_params, float tokens_per_sec, double step_seconds, int64_t total_tokens);
    AnomalyType classify() const;

    std::vector<Record> ring_;  // the last `window` steps
    size_t head_ = 0, size_ = 0;
    Ema loss_short_, loss_long_, grad_;
    TelemetrySnapshot latest_;
};

}  // namespace aic
