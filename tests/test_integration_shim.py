"""The reference-side shim of the integration guide (its block marked `shim:compile`) compiles, and the
library's status codes keep the reference's ErrorCode numbering, so the shim can forward a
code with a cast.

The shim is compiled with g++ -fsyntax-only against include/aic_hip.h and a minimal
declaration of the reference's error interface -- the names and signatures the shim uses
(aic::ErrorCode, aic::detail::str_cat, aic::detail::throw_error, AIC_THROW;
include/core/error.hpp:13-75 of the reference) -- written here, not copied; nothing of the
reference is built.  CPU only."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# include/core/error.hpp:13-29 of the reference: InvalidArgument = 1, then in order
REFERENCE_CODES = ["InvalidArgument", "OutOfRange", "ShapeMismatch", "DTypeMismatch", "DeviceMismatch", "OutOfMemory",
                   "CudaError", "NotImplemented", "BackendUnavailable", "IOError", "FormatError", "Overflow",
                   "InvalidState", "RuntimeError", "Internal"]

ERROR_INTERFACE = """#pragma once
#include <sstream>
#include <string>
using cudaStream_t = void*;
namespace aic {
enum class ErrorCode : int { %s };
namespace detail {
template <typename... Args>
std::string str_cat(const Args&... args) { std::ostringstream os; (os << ... << args); return os.str(); }
[[noreturn]] void throw_error(ErrorCode code, const std::string& message, const char* file, int line);
}  // namespace detail
}  // namespace aic
#define AIC_THROW(code, ...) \\
    ::aic::detail::throw_error(::aic::ErrorCode::code, ::aic::detail::str_cat(__VA_ARGS__), __FILE__, __LINE__)
""" % ", ".join([f"{REFERENCE_CODES[0]} = 1"] + REFERENCE_CODES[1:])


def shim_block():
    guide = os.path.join(ROOT, "INTEGRATION.md")
    text = open(guide).read()
    m = re.search(r"<!-- shim:compile -->\s*```cpp\n(.*?)```", text, re.S)
    assert m, f"{guide} has no block marked shim:compile"
    return m.group(1)


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_integration_shim_compiles(tmp_path):
    inc = tmp_path / "core"
    inc.mkdir()
    (inc / "error.hpp").write_text(ERROR_INTERFACE)
    src = tmp_path / "aic_hip_backend.cpp"
    src.write_text(shim_block())
    p = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-Werror", "-I", str(tmp_path), "-I",
                        os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
    assert p.returncode == 0, p.stderr


def test_shim_defines_the_reference_launchers():
    code = shim_block()
    for name in ("launch_flash_attention_forward_gpu", "launch_flash_attention_backward_gpu",
                 "cuda_cross_entropy_forward", "cuda_cross_entropy_backward", "cuda_adamw_step",
                 "cuda_embedding_forward", "cuda_embedding_backward", "launch_dequantize_int4",
                 "launch_has_nan_or_inf_gpu", "launch_unscale_gpu"):
        assert re.search(r"\b" + name + r"\(", code), name


def test_library_error_codes_keep_the_reference_numbering():
    """csrc/runtime/error.hpp's ErrorCode: Ok = 0, then the reference's codes from 1 in order,
    with HipError in the reference's CudaError slot (7)."""
    text = open(os.path.join(ROOT, "autonomousaicore_amd", "csrc", "runtime", "error.hpp")).read()
    body = re.search(r"enum class ErrorCode : int \{(.*?)\};", text, re.S).group(1)
    names = [re.sub(r"\s*=.*", "", n).strip() for n in body.split(",") if n.strip()]
    assert names[0] == "Ok" and "InvalidArgument = 1" in body
    assert names[1:] == [("HipError" if n == "CudaError" else n) for n in REFERENCE_CODES]
