// Error policy of the library: C++ exceptions inside, integer status codes at the C-ABI.
// The codes keep the numbering of the reference's aic::ErrorCode
// (include/core/error.hpp:13-29) so a caller can map them back one to one; the reference's
// CudaError slot (7) is HipError here.
#pragma once

#include <sstream>
#include <stdexcept>
#include <string>

namespace aic {

enum class ErrorCode : int {
    Ok = 0,
    InvalidArgument = 1,
    OutOfRange,
    ShapeMismatch,
    DTypeMismatch,
    DeviceMismatch,
    OutOfMemory,
    HipError,
    NotImplemented,
    BackendUnavailable,
    IOError,
    FormatError,
    Overflow,
    InvalidState,
    RuntimeError,
    Internal
};

const char* error_code_name(ErrorCode c) noexcept;

class Error : public std::runtime_error {
public:
    Error(ErrorCode code, const std::string& msg, const char* file, int line)
        : std::runtime_error(format(code, msg, file, line)), code_(code) {}
    ErrorCode code() const noexcept { return code_; }

private:
    static std::string format(ErrorCode code, const std::string& msg, const char* file, int line) {
        std::ostringstream os;
        os << "[" << error_code_name(code) << "] " << msg << " (" << file << ":" << line << ")";
        return os.str();
    }
    ErrorCode code_;
};

namespace detail {
template <typename... Args>
std::string cat(const Args&... args) {
    std::ostringstream os;
    (os << ... << args);
    return os.str();
}
}  // namespace detail

}  // namespace aic

#define AIC_THROW(code, ...) \
    throw ::aic::Error(::aic::ErrorCode::code, ::aic::detail::cat(__VA_ARGS__), __FILE__, __LINE__)

#define AIC_CHECK(cond, code, ...)                                                                 \
    do {                                                                                           \
        if (!(cond))                                                                               \
            throw ::aic::Error(::aic::ErrorCode::code,                                             \
                               ::aic::detail::cat("check failed: (" #cond ") ", ##__VA_ARGS__),   \
                               __FILE__, __LINE__);                                                \
    } while (false)

#define AIC_HIP_CHECK(expr)                                                                        \
    do {                                                                                           \
        hipError_t _st = (expr);                                                                   \
        if (_st != hipSuccess)                                                                     \
            throw ::aic::Error(::aic::ErrorCode::HipError,                                         \
                               ::aic::detail::cat(#expr, " -> ", hipGetErrorString(_st)),          \
                               __FILE__, __LINE__);                                                \
    } while (false)
