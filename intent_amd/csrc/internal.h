// Host-side helpers shared by the entry points (error state, checks).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/intent_amd.h"

namespace intent {

// Records a formatted message for intent_amd_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread's error message.
void clear_error();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// rows * stride_bytes stays below 2^31: the byte offsets of buffer loads are
// 32-bit and the kernels keep them non-negative ints.
inline bool fits_offset(int64_t rows, int64_t stride_bytes) {
  return rows >= 0 && stride_bytes >= 0 && (rows == 0 || stride_bytes <= ((int64_t)1 << 31) / rows) &&
         rows * stride_bytes < ((int64_t)1 << 31);
}

// Checks hipGetLastError() after a launch and records `kernel` as the
// thread's last launched kernel (intent_amd_last_kernel()).
int launch_status(const char* kernel);
// Same, with a printf-formatted kernel name (template parameters).
int launch_status_fmt(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Writes `bits` (the low elem_bytes = 1, 2 or 4 bytes) to every element of a
// rows x cols matrix with a leading stride of ld elements: the output of a
// contraction over an empty K, which is its epilogue applied to zero.
int fill_launch(void* out, int64_t rows, int64_t cols, int64_t ld, int elem_bytes, uint32_t bits, void* stream);

// Compute units of the current device (queried once per device; 0 if the
// query fails, which callers treat as "no round-fitting").
int cu_count();

}  // namespace intent

#define INTENT_REQUIRE(cond, code, ...)            \
  do {                                             \
    if (!(cond)) return ::intent::fail(code, __VA_ARGS__); \
  } while (0)
