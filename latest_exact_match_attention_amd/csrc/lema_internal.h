// Shared host/device helpers of liblema_hip.so. Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/lema_hip.h"

namespace lema {

// The thread-local message behind lema_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Check a HIP call made by a launcher; on failure record the message and return the status.
#define LEMA_HIP_CHECK(expr)                                                              \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess) {                                                               \
      ::lema::set_error("%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
      return LEMA_HIP_ERROR;                                                              \
    }                                                                                     \
  } while (0)

#define LEMA_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::lema::set_error(__VA_ARGS__);    \
      return LEMA_BAD_ARG;               \
    }                                    \
  } while (0)

// After a launch: report a launch failure (bad configuration, missing code object).
inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("launch of %s failed: %s", what, hipGetErrorString(e));
    return LEMA_HIP_ERROR;
  }
  return LEMA_OK;
}

inline int dtype_size(int32_t dtype) {
  switch (dtype) {
    case LEMA_F32: return 4;
    case LEMA_F16: return 2;
    case LEMA_BF16: return 2;
    default: return 0;
  }
}

inline bool aligned(const void* p, int64_t a) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(a)) == 0;
}

// Exact 32-bit division by a runtime divisor d >= 1 (Lemire, Kaser and Kurz, "Faster
// remainder by direct computation", 2019): q = hi64(M * n) with M = floor((2^64 - 1) / d) + 1,
// exact for every 32-bit n and d >= 2; d = 1 (where M would wrap to 0) is passed through.
struct FastDiv {
  uint64_t m;
  uint32_t d;
  FastDiv() = default;
  explicit FastDiv(uint32_t div) : m(div > 1 ? ~0ULL / div + 1 : 0), d(div) {}
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return d == 1 ? n : static_cast<uint32_t>(__umul64hi(m, static_cast<uint64_t>(n)));
  }
};

// MI355X dispatches consecutive workgroups round-robin over its 8 XCDs, each with its own
// 4 MB L2; kernels map blockIdx so that work sharing data lands on one XCD.
constexpr int kNumXcd = 8;

// Clang vector types: __builtin_nontemporal_store needs these rather than HIP's structs.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

}  // namespace lema
