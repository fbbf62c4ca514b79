#pragma once

#include <cstdint>

namespace aic::data {

uint64_t splitmix64(uint64_t x);
void uniform_ids(uint64_t seed, int64_t n, int64_t vocab, int64_t* out);
void zipf_ids(uint64_t seed, int64_t n, int64_t vocab, double s, int64_t* out);
void normal(uint64_t seed, int64_t n, float mean, float std, float* out);

}  // namespace aic::data
