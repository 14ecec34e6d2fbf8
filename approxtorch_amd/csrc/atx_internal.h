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
// Records the caller's timing event (atx_set_timing_events) on the stream:
// `after` false = before the LUT GEMM's main kernel, true = after it.
int timing_mark(bool after, hipStream_t stream);

inline long long cdiv(long long a, long long b) { return (a + b - 1) / b; }

// Validates a conv geometry (sizes, strides, OH/OW consistent); ATX_OK or
// ATX_EINVAL with a message.
int check_geom(const atx_conv_geom& g);

// out[i] = sum_s ws[s*numel + i] in a fixed order (deterministic), with the
// optional per-channel fake-quant STE out = (mask ? sum : 0) / max(scale[i/K],
// 1e-12); S = 0 writes zeros.  zsum (nullable, with zsx, zzx and scale):
// before the STE, out -= (zsum[o] * (zsx[0] * scale[o])) * zzx[0], each
// operation rounded on its own (the uint8 layer's weight zero-point term).
int launch_split_sum(const float* ws, int S, long long numel, int K, const uint8_t* mask,
                     const float* scale, float* out, hipStream_t stream,
                     const float* zsum = nullptr, const float* zsx = nullptr,
                     const float* zzx = nullptr);

// fp32-class LUT GEMM (ascending-k fp32 sums, tiled over LDS tables built
// from the transposed fp32 LUT image); out_kind ATX_OUT_F32 or
// ATX_OUT_DEQUANT.  Arguments validated by atx_lut_gemm.
int lut_gemm_f32_tiled(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                       const float* lutf32t, int N, int K, int L, int O, int out_kind,
                       const float* sx, const float* sw, const float* bias, float* y,
                       hipStream_t stream);

// The uint8 layer's zero-point correction and dequant as an epilogue
// (atx_lut_gemm_narrow_uint8): for the sum v = (float) y[n,o,l],
//   t = v - zw[o] * xs[n*L + l];  t = t - zx * ws[o];  t = t + (K * zx) * zw[o];
//   out = bias ? bias[o] + t * (sx * sw[o]) : t * (sx * sw[o])
// with each operation in fp32 in that order, the same roundings as
// atx_uint8_dequant applied to the fp32 sums.
constexpr int OUT_DEQUANT_U8 = 3;
struct U8Terms {
  const float* xs; const float* ws; const float* zx; const float* zw;
  float K;
};
__device__ __forceinline__ float u8_dequant(float v, float x, float zo, float wo, float ko,
                                            float so, const float* bias, float bo) {
  float t = v - zo * x;
  t = t - wo;
  t = t + ko;
  t = t * so;
  return bias ? bo + t : t;
}

// Sum of S int32 partial slices of an [N][O][L] LUT GEMM output (ws[s *
// numel + i], exact in int64) followed by the epilogue ep into y
// (ep.out_kind may be OUT_DEQUANT_U8, with its terms in u8).
int launch_split_reduce(const int* ws, int S, long long numel, int O, int L,
                        const atx_gemm_epilogue& ep, void* y, hipStream_t stream,
                        const U8Terms& u8 = U8Terms{});

// Grid size for grid-stride elementwise kernels.
inline int elem_grid(long long n, int threads, int cap = 8192) {
  long long b = cdiv(n, threads);
  if (b < 1) b = 1;
  return (int)(b < cap ? b : cap);
}

// Remainder of v after its truncated bf16 high part h (the bits of v with
// the low 16 cleared): v - h, exact for finite v.  For +-inf and NaN the
// high part already is the whole value (inf, or a NaN), so the remainder is
// 0 instead of the NaN that inf - inf gives.
__device__ __forceinline__ float bf16_rest(float v) {
  const float r = v - __uint_as_float(__float_as_uint(v) & 0xffff0000u);
  return __builtin_isfinite(v) ? r : 0.0f;
}

// Byte offset of row v in the LUT GEMM's LDS tables (256-byte lines holding
// row v of four tables; within a table's 64-byte quarter, chunk g of row v
// sits at position g ^ ((v >> 1) & 3)).
__device__ __forceinline__ unsigned row_offset(unsigned v) {
  return v * 256u + (((v >> 1) & 3u) << 4);
}

// Row-offset operand layout of the LUT GEMM: the k-rows come in quads
// (Kpad = K rounded up to 4 rows); slot s of a quad holds, for row r, tap
// k = (s & ~3) | (((r >> 2) + s) & 3), so that the GEMM's row group reading
// quarter ((r >> 2) + s) & 3 at sub-step s finds its tap in slot s.  Taps at
// or beyond K hold offset 0.
__host__ __device__ __forceinline__ int operand_tap(int slot, int r) {
  return (slot & ~3) | (((r >> 2) + slot) & 3);
}
__host__ __device__ __forceinline__ int operand_slot(int k, int r) {
  return (k & ~3) | ((k - (r >> 2)) & 3);
}
__host__ __device__ __forceinline__ int operand_rows(int K) { return (K + 3) & ~3; }

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

// First check of every entry point taking an atx_gemm_epilogue: its size
// field must be this header's sizeof (an older caller's struct is rejected).
#define ATX_REQUIRE_EPILOGUE(ep, fn)                                              \
  ATX_REQUIRE((ep).size == (int)sizeof(atx_gemm_epilogue),                        \
              fn ": atx_gemm_epilogue.size is %d, expected %d (caller built "     \
              "against another atx.h; ABI version %d)", (ep).size,                \
              (int)sizeof(atx_gemm_epilogue), ATX_ABI_VERSION)
