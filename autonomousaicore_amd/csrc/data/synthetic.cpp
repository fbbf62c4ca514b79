// Counter-based synthetic inputs (splitmix64): uniform and Zipf token ids and N(mean, std)
// weights.  Every value depends only on (seed, index), so any slice can be regenerated
// independently and in parallel.  The reference draws from a thread_local
// std::mt19937(1337) (src/tensor/tensor.cpp:508-540), whose normal stream is
// implementation-defined; weights are therefore exchanged explicitly, never re-derived.
#include "synthetic.hpp"

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

namespace aic::data {

uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// 53-bit uniform in [0, 1).
static double u01(uint64_t key, uint64_t c) { return static_cast<double>(splitmix64(key ^ c) >> 11) * 0x1.0p-53; }

void uniform_ids(uint64_t seed, int64_t n, int64_t vocab, int64_t* out) {
    const uint64_t key = splitmix64(seed);
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t r = splitmix64(key ^ static_cast<uint64_t>(i));
        out[i] = static_cast<int64_t>(((r >> 32) * static_cast<uint64_t>(vocab)) >> 32);
    }
}

void zipf_ids(uint64_t seed, int64_t n, int64_t vocab, double s, int64_t* out) {
    std::vector<double> cdf(static_cast<size_t>(vocab));
    double acc = 0.0;
    for (int64_t k = 1; k <= vocab; ++k) {
        acc += std::pow(static_cast<double>(k), -s);
        cdf[static_cast<size_t>(k - 1)] = acc;
    }
    const uint64_t key = splitmix64(seed);
    for (int64_t i = 0; i < n; ++i) {
        const double u = u01(key, static_cast<uint64_t>(i)) * acc;
        const auto it = std::upper_bound(cdf.begin(), cdf.end(), u);
        int64_t id = static_cast<int64_t>(it - cdf.begin());
        if (id >= vocab) id = vocab - 1;
        out[i] = id;
    }
}

void normal(uint64_t seed, int64_t n, float mean, float std, float* out) {
    const uint64_t key = splitmix64(seed);
    const int64_t nth = std::max<int64_t>(1, std::min<int64_t>(16, n / (1 << 20)));
    auto work = [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; ++i) {
            const uint64_t c = static_cast<uint64_t>(i);
            const double u1 = (static_cast<double>(splitmix64(key ^ (2 * c)) >> 11) + 1.0) * 0x1.0p-53;
            const double u2 = static_cast<double>(splitmix64(key ^ (2 * c + 1)) >> 11) * 0x1.0p-53;
            const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
            out[i] = mean + std * static_cast<float>(z);
        }
    };
    if (nth == 1) {
        work(0, n);
        return;
    }
    std::vector<std::thread> th;
    const int64_t chunk = (n + nth - 1) / nth;
    for (int64_t t = 0; t < nth; ++t) th.emplace_back(work, t * chunk, std::min(n, (t + 1) * chunk));
    for (auto& t : th) t.join();
}

}  // namespace aic::data
