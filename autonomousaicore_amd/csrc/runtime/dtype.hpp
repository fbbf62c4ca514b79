// Element types.  The numeric values are those of the reference's aic::DType
// (include/core/dtype.hpp:18-26), which is also what its .aic checkpoints store.
#pragma once

#include <cstddef>
#include <cstdint>

namespace aic {

enum class DType : std::uint8_t {
    Float32 = 0,
    Float16 = 1,
    BFloat16 = 2,
    Int32 = 3,
    Int64 = 4,
    UInt8 = 5,
    UInt16 = 6
};

constexpr std::size_t dtype_size(DType d) noexcept {
    switch (d) {
        case DType::Float32: return 4;
        case DType::Float16: return 2;
        case DType::BFloat16: return 2;
        case DType::Int32: return 4;
        case DType::Int64: return 8;
        case DType::UInt8: return 1;
        case DType::UInt16: return 2;
    }
    return 0;
}

const char* dtype_name(DType d) noexcept;

}  // namespace aic
