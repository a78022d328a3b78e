// Internal helpers for the extern "C" entry points: error reporting and checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <string>

#include "../../include/thintensor_hip.h"

namespace tt {

void set_error(const char* fmt, ...);

#define TT_REQUIRE(cond, ...)                 \
  do {                                        \
    if (!(cond)) {                            \
      ::tt::set_error(__VA_ARGS__);           \
      return TT_ERR_INVALID;                  \
    }                                         \
  } while (0)

#define TT_UNSUPPORTED(cond, ...)             \
  do {                                        \
    if (!(cond)) {                            \
      ::tt::set_error(__VA_ARGS__);           \
      return TT_ERR_UNSUPPORTED;              \
    }                                         \
  } while (0)

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return TT_ERR_HIP;
  }
  return TT_OK;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// y[r] = W x[r] + bias for m fp16 activation rows through the GEMV engine, several rows
// per launch sharing every weight load; row r has the bits of the single-row GEMV + bias
// (batched.hip).  Shapes and alignment checked by the caller.
int dense_bias_rows_f16(const void* weight, int64_t w_row, const void* bias, const void* x, int64_t x_row, void* out,
                        int64_t out_row, int64_t m, int64_t rows, int64_t cols, hipStream_t st);

// Expert index arrays are int32 or int64 (index_bytes 4 or 8); the kernels take the
// log2 of the size in 32-bit words.
inline bool index_shift(int index_bytes, int* shift) {
  *shift = index_bytes == 8 ? 1 : 0;
  return index_bytes == 4 || index_bytes == 8;
}

inline bool valid_act_dtype(int d) { return d == TT_F16 || d == TT_BF16; }
inline bool valid_out_dtype(int d) { return d == TT_F16 || d == TT_BF16 || d == TT_F32; }

// Attention scratch: kAttnCounters arrival counters of the single-launch path (one per
// KV head, at fixed offsets whatever the shape, left at zero by every call), then the
// chunk partials (m, l, o) per query head.
constexpr int kAttnCounters = 1024;

}  // namespace tt
