// Test-only restatement of the reference's runtime error types
// (include/kernelh/runtime/runtime_error.hpp:20-31): the declarations the
// Backend binding compiles against, nothing more. Result<T> is
// std::expected<T, Error>; this image's C++ library (GCC 11) has no
// <expected>, so expected_subset.hpp supplies the part of it the binding
// uses when the library lacks it.
#ifndef KH_RESTATED_RUNTIME_ERROR_HPP
#define KH_RESTATED_RUNTIME_ERROR_HPP

#if __has_include(<expected>) && __cplusplus > 202002L
#include <expected>
#else
#include "expected_subset.hpp"
#endif
#include <string>

namespace kernelh::runtime {

inline constexpr int kCudaDriverUnavailable = 77;

struct Error {
  int code = 0;
  std::string message;
  bool is_success() const { return code == 0; }
};

template <typename T>
using Result = std::expected<T, Error>;

}  // namespace kernelh::runtime

#endif
