#include "telemetry.hpp"

#include <hip/hip_runtime.h>

#include <cmath>
#include <fstream>
#include <sstream>
#include <string>

namespace aic {

const char* anomaly_name(AnomalyType t) {
    static const char* const names[] = {"None",           "NanOrInfLoss",      "NanOrInfGradient", "LossDivergence",
                                        "GradientExplosion", "GradientVanishing", "MemoryCritical"};
    const int i = static_cast<int>(t);
    return (i >= 0 && i < static_cast<int>(sizeof(names) / sizeof(names[0]))) ? names[i] : "Unknown";
}

std::string TelemetrySnapshot::to_json() const {
    std::ostringstream os;
    auto field = [&os](const char* key, auto value, bool last = false) {
        os << '"' << key << "\":" << value << (last ? "" : ",");
    };
    os << '{';
    field("step", step);
    field("loss", loss);
    field("loss_ema_short", loss_ema_short);
    field("loss_ema_long", loss_ema_long);
    field("loss_variance", loss_variance);
    field("grad_norm", grad_norm);
    field("grad_norm_ema", grad_norm_ema);
    field("lr", lr);
    field("tokens_per_sec", tokens_per_sec);
    field("estimated_tflops", estimated_tflops);
    field("host_total_bytes", memory.host_total);
    field("host_free_bytes", memory.host_free);
    field("gpu_total_bytes", memory.gpu_total);
    field("gpu_free_bytes", memory.gpu_free);
    os << "\"anomaly\":\"" << anomaly_name(anomaly) << "\"}";
    return os.str();
}

void TelemetryTracker::Ema::add(float x) {
    if (!std::isfinite(x)) return;
    value = seeded ? alpha * value + (1.0f - alpha) * x : x;
    seeded = true;
}

TelemetryTracker::TelemetryTracker(size_t window, float alpha_short, float alpha_long)
    : ring_(window > 0 ? window : 1), loss_short_{alpha_short}, loss_long_{alpha_long}, grad_{alpha_short} {}

const TelemetryTracker::Record& TelemetryTracker::from_newest(size_t i) const {
    return ring_[(head_ + ring_.size() - 1 - i) % ring_.size()];
}

HardwareMemoryStats TelemetryTracker::query_memory(int device_index) {
    HardwareMemoryStats m;
    std::ifstream meminfo("/proc/meminfo");
    std::string key, unit;
    unsigned long long kib = 0;
    while (meminfo >> key >> kib >> unit) {
        if (key == "MemTotal:") m.host_total = kib << 10;
        else if (key == "MemAvailable:") m.host_free = kib << 10;
    }
    int count = 0, current = 0;
    if (device_index >= 0 && hipGetDeviceCount(&count) == hipSuccess && device_index < count &&
        hipGetDevice(&current) == hipSuccess) {
        size_t free_b = 0, total_b = 0;
        if (hipSetDevice(device_index) == hipSuccess && hipMemGetInfo(&free_b, &total_b) == hipSuccess) {
            m.gpu_free = free_b;
            m.gpu_total = total_b;
        }
        (void)hipSetDevice(current);
    }
    (void)hipGetLastError();  // a failed query leaves no sticky error behind
    return m;
}

TelemetrySnapshot TelemetryTracker::record_step(int64_t step, float loss, float grad_norm, float lr,
                                                float tokens_per_sec, double step_seconds, int64_t total_tokens,
                                                int64_t model_params, int device_index) {
    loss_short_.add(loss);
    loss_long_.add(loss);
    grad_.add(grad_norm);

    ring_[head_] = Record{loss, grad_norm, loss_long_.value};
    head_ = (head_ + 1) % ring_.size();
    if (size_ < ring_.size()) ++size_;

    TelemetrySnapshot s;
    s.step = step;
    s.loss = loss;
    s.grad_norm = grad_norm;
    s.lr = lr;
    s.tokens_per_sec = tokens_per_sec;
    s.loss_ema_short = loss_short_.value;
    s.loss_ema_long = loss_long_.value;
    s.grad_norm_ema = grad_.value;
    s.loss_variance = window_loss_variance();
    s.estimated_tflops = tflops(model_params, tokens_per_sec, step_seconds, total_tokens);
    s.memory = query_memory(device_index);
    latest_ = s;
    latest_.anomaly = classify();
    return latest_;
}

float TelemetryTracker::window_loss_variance() const {
    // population variance of the finite losses in the window, two passes in double
    double sum = 0.0;
    size_t n = 0;
    for (size_t i = 0; i < size_; ++i)
        if (std::isfinite(from_newest(i).loss)) {
            sum += from_newest(i).loss;
            ++n;
        }
    if (n < 2) return 0.0f;
    const double mean = sum / static_cast<double>(n);
    double dev2 = 0.0;
    for (size_t i = 0; i < size_; ++i)
        if (std::isfinite(from_newest(i).loss)) {
            const double d = from_newest(i).loss - mean;
            dev2 += d * d;
        }
    return static_cast<float>(dev2 / static_cast<double>(n));
}

float TelemetryTracker::tflops(int64_t model_params, float tokens_per_sec, double step_seconds, int64_t total_tokens) {
    // 6 FLOP per parameter per token (forward 2, backward 4)
    if (model_params <= 0) return 0.0f;
    double tps = tokens_per_sec;
    if (tps <= 0.0 && step_seconds > 0.0 && total_tokens > 0) tps = static_cast<double>(total_tokens) / step_seconds;
    return tps > 0.0 ? static_cast<float>(6.0 * static_cast<double>(model_params) * tps / 1e12) : 0.0f;
}

AnomalyType TelemetryTracker::classify() const {
    if (!std::isfinite(latest_.loss)) return AnomalyType::NanOrInfLoss;
    if (!std::isfinite(latest_.grad_norm)) return AnomalyType::NanOrInfGradient;
    if (is_diverging()) return AnomalyType::LossDivergence;
    if (is_gradient_exploding()) return AnomalyType::GradientExplosion;
    if (is_gradient_vanishing()) return AnomalyType::GradientVanishing;
    if (is_memory_critical()) return AnomalyType::MemoryCritical;
    return AnomalyType::None;
}

bool TelemetryTracker::is_nan_or_inf() const {
    return !std::isfinite(latest_.loss) || !std::isfinite(latest_.grad_norm);
}

bool TelemetryTracker::is_diverging(float threshold_ratio, int min_consecutive) const {
    // the newest min_consecutive records (at least 3 in the window) each had a finite loss above
    // threshold_ratio times the long EMA of its own step
    if (size_ < 3 || min_consecutive < 1 || static_cast<size_t>(min_consecutive) > size_) return false;
    for (int i = 0; i < min_consecutive; ++i) {
        const Record& r = from_newest(static_cast<size_t>(i));
        if (!std::isfinite(r.loss) || !(r.loss_ema_long > 1e-6f) || !(r.loss > threshold_ratio * r.loss_ema_long))
            return false;
    }
    return true;
}

bool TelemetryTracker::is_gradient_exploding(float spike_factor) const {
    if (size_ < 5) return false;
    // against the gradient EMA (which already includes this step); an absolute bound when the
    // EMA is too small to compare against
    return grad_.value > 1e-6f ? latest_.grad_norm > spike_factor * grad_.value : latest_.grad_norm > 100.0f;
}

bool TelemetryTracker::is_gradient_vanishing(float min_norm) const {
    return size_ >= 5 && latest_.grad_norm < min_norm;
}

bool TelemetryTracker::is_memory_critical(float min_free_ratio) const {
    const HardwareMemoryStats& m = latest_.memory;
    return m.gpu_total > 0 &&
           static_cast<double>(m.gpu_free) < static_cast<double>(min_free_ratio) * static_cast<double>(m.gpu_total);
}

void TelemetryTracker::reset() {
    for (Ema* e : {&loss_short_, &loss_long_, &grad_}) *e = Ema{e->alpha};
    head_ = size_ = 0;
    latest_ = TelemetrySnapshot{};
}

}  // namespace aic
