// SPDX-License-Identifier: MIT
// Host-side plumbing shared by every C-ABI entry point: error reporting,
// argument checks that run before any HIP call (so they work without a GPU),
// the gfx950 arch gate and launch-error capture.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/strix_amd.h"

namespace strix {

// Records `fmt` as this thread's last error and returns STRIX_ERR_INVALID.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// 0 when the current device is gfx950, else an error (message set).
int check_arch();

// Compute units of the current device (cached; 256 if the query fails).
// Called after check_arch() has passed.
int cu_count();

// Captures a launch error (if any) into the error slot.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// The tiled kernels address an operand's rows with 32-bit per-lane byte
// offsets from a wave-uniform base: true when `rows` rows of `row_bytes`
// bytes at a stride of `stride_bytes` all lie within 4 GiB of the first.
inline bool fits_u32_rows(int64_t rows, int64_t stride_bytes, int64_t row_bytes) {
  return rows <= 0 || (rows - 1) * stride_bytes + row_bytes <= (int64_t)UINT32_MAX;
}

}  // namespace strix

// Validation helpers: return from the enclosing entry point with a message.
#define STRIX_REQUIRE(cond, ...)                                  \
  do {                                                            \
    if (!(cond)) return ::strix::set_error(STRIX_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define STRIX_ARCH_GATE()                       \
  do {                                          \
    int _rc = ::strix::check_arch();            \
    if (_rc != STRIX_OK) return _rc;            \
  } while (0)
