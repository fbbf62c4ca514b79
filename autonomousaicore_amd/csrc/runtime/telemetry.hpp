// Step telemetry and anomaly detection (TelemetryTracker, include/autonomous/telemetry.hpp,
// src/autonomous/telemetry.cpp:126-275): per-step loss / gradient-norm EMAs, the rolling
// loss variance over a window, TFLOP/s from 6 P tokens/s, host and GPU memory, and the
// reference's anomaly rules (non-finite loss or gradient, loss divergence above 1.4x the long
// EMA for 3 steps, gradient spikes above 4x the gradient EMA, vanishing gradients, GPU memory
// under 8% free).  The step statistics it consumes come from the device-side step history of
// TransformerLM, read in batches, so the training loop needs no host synchronisation per step.
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>
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
    size_t count() const { return history_.size(); }
    const TelemetrySnapshot& latest() const { return latest_; }
    void reset();

private:
    size_t window_;
    float a_short_, a_long_;
    float ema_s_ = 0.0f, ema_l_ = 0.0f, gn_ema_ = 0.0f;
    int consecutive_ = 0;
    std::deque<TelemetrySnapshot> history_;
    TelemetrySnapshot latest_;
};

}  // namespace aic
