// Internal helpers shared by the HIP translation units of libatx.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/atx.h"

namespace atx {

// Records a message for atx_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);

// Checks the launch that was just issued (hipGetLastError) and converts a
// failure into ATX_ELAUNCH with the kernel's name in the message.
int check_launch(const char* what);

inline long long cdiv(long long a, long long b) { return (a + b - 1) / b; }

// Grid size for grid-stride elementwise kernels.
inline int elem_grid(long long n, int threads, int cap = 8192) {
  long long b = cdiv(n, threads);
  if (b < 1) b = 1;
  return (int)(b < cap ? b : cap);
}

// Byte offset of row v of a LUT GEMM table (128-byte rows of 8 16-byte
// channel chunks; chunk g of row v sits at position g ^ ((v >> 1) & 7)).
__device__ __forceinline__ unsigned row_offset(unsigned v) {
  return v * 128u + (((v >> 1) & 7u) << 4);
}

// clamp(rint(v) + offset, 0, 255) with round-half-even; NaN maps to `offset`
// clamped (the reference's float->int conversion of NaN is unspecified).
__device__ __forceinline__ unsigned quant_index(float v, int offset) {
  float r = __builtin_rintf(v);
  int q = (r == r) ? (int)fminf(fmaxf(r, -1024.f), 1024.f) : 0;
  q += offset;
  q = q < 0 ? 0 : (q > 255 ? 255 : q);
  return (unsigned)q;
}

}  // namespace atx

#define ATX_REQUIRE(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return ::atx::set_error(ATX_EINVAL, __VA_ARGS__); \
  } while (0)
