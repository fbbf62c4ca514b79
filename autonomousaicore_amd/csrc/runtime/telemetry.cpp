#include "telemetry.hpp"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <sstream>

namespace aic {

const char* anomaly_name(AnomalyType t) {
    switch (t) {
        case AnomalyType::None: return "None";
        case AnomalyType::NanOrInfLoss: return "NanOrInfLoss";
        case AnomalyType::NanOrInfGradient: return "NanOrInfGradient";
        case AnomalyType::LossDivergence: return "LossDivergence";
        case AnomalyType::GradientExplosion: return "GradientExplosion";
        case AnomalyType::GradientVanishing: return "GradientVanishing";
        case AnomalyType::MemoryCritical: return "MemoryCritical";
    }
    return "Unknown";
}

std::string TelemetrySnapshot::to_json() const {
    std::ostringstream os;
    os << "{\"step\":" << step << ",\"loss\":" << loss << ",\"loss_ema_short\":" << loss_ema_short
       << ",\"loss_ema_long\":" << loss_ema_long << ",\"loss_variance\":" << loss_variance
       << ",\"grad_norm\":" << grad_norm << ",\"grad_norm_ema\":" << grad_norm_ema << ",\"lr\":" << lr
       << ",\"tokens_per_sec\":" << tokens_per_sec << ",\"estimated_tflops\":" << estimated_tflops
       << ",\"host_total_bytes\":" << memory.host_total << ",\"host_free_bytes\":" << memory.host_free
       << ",\"gpu_total_bytes\":" << memory.gpu_total << ",\"gpu_free_bytes\":" << memory.gpu_free
       << ",\"anomaly\":\"" << anomaly_name(anomaly) << "\"}";
    return os.str();
}

TelemetryTracker::TelemetryTracker(size_t window, float alpha_short, float alpha_long)
    : window_(window > 0 ? window : 1), a_short_(alpha_short), a_long_(alpha_long) {}

HardwareMemoryStats TelemetryTracker::query_memory(int device_index) {
    HardwareMemoryStats m;
    if (std::FILE* f = std::fopen("/proc/meminfo", "r")) {
        char key[64];
        unsigned long long kb = 0;
        char unit[16];
        while (std::fscanf(f, "%63s %llu %15s", key, &kb, unit) == 3) {
            if (std::strcmp(key, "MemTotal:") == 0) m.host_total = kb * 1024ull;
            if (std::strcmp(key, "MemAvailable:") == 0) m.host_free = kb * 1024ull;
        }
        std::fclose(f);
    }
    if (device_index >= 0) {
        int n = 0, cur = 0;
        if (hipGetDeviceCount(&n) == hipSuccess && device_index < n && hipGetDevice(&cur) == hipSuccess) {
            size_t fr = 0, tot = 0;
            if (hipSetDevice(device_index) == hipSuccess && hipMemGetInfo(&fr, &tot) == hipSuccess) {
                m.gpu_free = fr;
                m.gpu_total = tot;
            }
            (void)hipSetDevice(cur);
        }
        (void)hipGetLastError();
    }
    return m;
}

TelemetrySnapshot TelemetryTracker::record_step(int64_t step, float loss, float grad_norm, float lr,
                                                float tokens_per_sec, double step_seconds, int64_t total_tokens,
                                                int64_t model_params, int device_index) {
    TelemetrySnapshot s;
    s.step = step;
    s.loss = loss;
    s.grad_norm = grad_norm;
    s.lr = lr;
    s.tokens_per_sec = tokens_per_sec;
    s.memory = query_memory(device_index);
    if (model_params > 0) {  // 6 P FLOP per token
        if (tokens_per_sec > 0.0f)
            s.estimated_tflops = static_cast<float>(6.0 * model_params * static_cast<double>(tokens_per_sec) / 1e12);
        else if (step_seconds > 0.0 && total_tokens > 0)
            s.estimated_tflops = static_cast<float>(6.0 * model_params * static_cast<double>(total_tokens) /
                                                    step_seconds / 1e12);
    }
    const bool loss_ok = std::isfinite(loss), gn_ok = std::isfinite(grad_norm);
    if (!loss_ok) s.anomaly = AnomalyType::NanOrInfLoss;
    else if (!gn_ok) s.anomaly = AnomalyType::NanOrInfGradient;
    if (history_.empty()) {
        ema_s_ = ema_l_ = loss;
        gn_ema_ = grad_norm;
    } else {
        if (loss_ok) {
            ema_s_ = a_short_ * ema_s_ + (1.0f - a_short_) * loss;
            ema_l_ = a_long_ * ema_l_ + (1.0f - a_long_) * loss;
        }
        if (gn_ok) gn_ema_ = a_short_ * gn_ema_ + (1.0f - a_short_) * grad_norm;
    }
    s.loss_ema_short = ema_s_;
    s.loss_ema_long = ema_l_;
    s.grad_norm_ema = gn_ema_;
    history_.push_back(s);
    if (history_.size() > window_) history_.pop_front();
    if (history_.size() >= 2) {  // population variance of the finite losses in the window
        double sum = 0.0, sq = 0.0;
        size_t n = 0;
        for (const auto& h : history_)
            if (std::isfinite(h.loss)) {
                sum += h.loss;
                sq += static_cast<double>(h.loss) * h.loss;
                ++n;
            }
        if (n >= 2) {
            const double mean = sum / static_cast<double>(n), var = sq / static_cast<double>(n) - mean * mean;
            s.loss_variance = var > 0.0 ? static_cast<float>(var) : 0.0f;
        }
    }
    consecutive_ = (loss_ok && ema_l_ > 1e-6f && loss > 1.4f * ema_l_) ? consecutive_ + 1 : 0;
    latest_ = s;
    if (s.anomaly == AnomalyType::None) {
        if (is_diverging()) s.anomaly = AnomalyType::LossDivergence;
        else if (is_gradient_exploding()) s.anomaly = AnomalyType::GradientExplosion;
        else if (is_gradient_vanishing()) s.anomaly = AnomalyType::GradientVanishing;
        else if (is_memory_critical()) s.anomaly = AnomalyType::MemoryCritical;
    }
    latest_ = s;
    history_.back() = s;
    return s;
}

bool TelemetryTracker::is_nan_or_inf() const { return !std::isfinite(latest_.loss) || !std::isfinite(latest_.grad_norm); }

bool TelemetryTracker::is_diverging(float threshold_ratio, int min_consecutive) const {
    if (history_.size() < 3) return false;
    if (std::fabs(threshold_ratio - 1.4f) < 1e-4f) return consecutive_ >= min_consecutive;
    return ema_l_ > 1e-6f && latest_.loss > threshold_ratio * ema_l_ && consecutive_ >= min_consecutive;
}

bool TelemetryTracker::is_gradient_exploding(float spike_factor) const {
    if (history_.size() < 5) return false;
    if (gn_ema_ > 1e-6f) return latest_.grad_norm > spike_factor * gn_ema_;
    return latest_.grad_norm > 100.0f;
}

bool TelemetryTracker::is_gradient_vanishing(float min_norm) const {
    return history_.size() >= 5 && latest_.grad_norm < min_norm;
}

bool TelemetryTracker::is_memory_critical(float min_free_ratio) const {
    if (latest_.memory.gpu_total == 0) return false;
    return static_cast<float>(latest_.memory.gpu_free) / static_cast<float>(latest_.memory.gpu_total) < min_free_ratio;
}

void TelemetryTracker::reset() {
    history_.clear();
    ema_s_ = ema_l_ = gn_ema_ = 0.0f;
    consecutive_ = 0;
    latest_ = TelemetrySnapshot{};
}

}  // namespace aic
