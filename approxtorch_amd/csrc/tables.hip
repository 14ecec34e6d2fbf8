// LUT files and gradient-table generators.
//
// atx_parse_text_table: the text format of multiplier LUTs and gradient
// tables (approxtorch/load_lut.py:5-55, README.md:55-62): numbers separated
// by whitespace, '#' starts a comment, as numpy.loadtxt reads them.
//
// atx_lre_tables (grad_lut.py:14-37): grad_a[y] = least-squares slope of the
// LUT column LUT[:, y] over the row operand values, grad_b[x] = slope of the
// row LUT[x, :] over the column operand values; operand value = index -
// offset (128 for int8, 0 for uint8).  Closed-form OLS in fp64 (the slope
// scipy.stats.linregress returns), rounded to fp32.
//
// atx_date_tables (grad_lut.py:39-142): along each line of the LUT, a
// (2h+1)-tap moving average for h <= i <= 255-h (identity elsewhere), then
// (s[i+1] - s[i-1]) / 2 for h < i < 255-h and (s[255] - s[0]) / 255
// elsewhere, all in fp32.  The window mean reproduces numpy's float32 mean
// (pairwise summation: sequential below 8 terms, eight interleaved partial
// sums up to 128, halves above), so the tables equal the numpy
// implementation's bit for bit.

#include "atx_internal.h"

#include <errno.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

namespace atx {

__global__ void lre_tables_kernel(const float* __restrict__ lut, int offset,
                                  float* __restrict__ grad_a, float* __restrict__ grad_b) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;    // 0..511
  if (t >= 512) return;
  const bool col = t < 256;                 // grad_a: column y = t; grad_b: row x = t - 256
  const int j = col ? t : t - 256;
  const double xm = 127.5 - offset;         // mean of the operand values
  double vm = 0.0;
  for (int i = 0; i < 256; ++i) vm += (double)lut[col ? i * 256 + j : j * 256 + i];
  vm /= 256.0;
  double sxy = 0.0, sxx = 0.0;
  for (int i = 0; i < 256; ++i) {
    const double dx = (double)(i - offset) - xm;
    sxy += dx * ((double)lut[col ? i * 256 + j : j * 256 + i] - vm);
    sxx += dx * dx;
  }
  (col ? grad_a : grad_b)[j] = (float)(sxy / sxx);
}

// numpy's float32 pairwise sum of a[0..n) (n <= 255 here).
__device__ float np_pairwise_sum(const float* a, int n) {
  if (n < 8) {
    float res = 0.0f;
    for (int i = 0; i < n; ++i) res += a[i];
    return res;
  }
  if (n <= 128) {
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int i = 8;
    for (; i < n - (n % 8); i += 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    }
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
  }
  int n2 = n / 2;
  n2 -= n2 % 8;
  // both halves are <= 128 terms for n <= 255
  const float* b = a + n2;
  const int m = n - n2;
  float s1, s2;
  {
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int i = 8;
    for (; i < n2 - (n2 % 8); i += 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    }
    s1 = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n2; ++i) s1 += a[i];
  }
  {
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = b[j];
    int i = 8;
    for (; i < m - (m % 8); i += 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] += b[i + j];
    }
    s2 = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < m; ++i) s2 += b[i];
  }
  return s1 + s2;
}

// One block (256 threads) per LUT line: blocks 0..255 are the columns
// (grad_a, derivative along the row operand), 256..511 the rows (grad_b).
__global__ void __launch_bounds__(256)
date_tables_kernel(const float* __restrict__ lut, int half_ws, float* __restrict__ grad_a,
                   float* __restrict__ grad_b) {
  __shared__ float line[256];
  __shared__ float sm[256];
  const int b = blockIdx.x, i = threadIdx.x;
  const bool col = b < 256;
  const int j = col ? b : b - 256;
  const int at = col ? i * 256 + j : j * 256 + i;
  line[i] = lut[at];
  __syncthreads();
  const int w = 2 * half_ws + 1;
  float s = line[i];
  if (i >= half_ws && i <= 255 - half_ws)
    s = np_pairwise_sum(line + i - half_ws, w) / (float)w;
  sm[i] = s;
  __syncthreads();
  float g;
  if (i > half_ws && i < 255 - half_ws) g = (sm[i + 1] - sm[i - 1]) / 2.0f;
  else g = (sm[255] - sm[0]) / 255.0f;
  (col ? grad_a : grad_b)[at] = g;
}

}  // namespace atx

using namespace atx;

extern "C" {

int atx_parse_text_table(const char* path, int integral, float* out, long long capacity,
                         long long* count) {
  ATX_REQUIRE(path && count && (capacity == 0 || out), "atx_parse_text_table: null pointer");
  FILE* f = fopen(path, "rb");
  if (!f) return set_error(ATX_EINVAL, "%s: %s", path, strerror(errno));
  long long n = 0;
  int lineno = 1;
  char buf[64];
  int c = fgetc(f);
  while (c != EOF) {
    if (c == '#') {                                 // comment to end of line
      while (c != EOF && c != '\n') c = fgetc(f);
      continue;
    }
    if (c == '\n') { ++lineno; c = fgetc(f); continue; }
    if (c == ' ' || c == '\t' || c == '\r' || c == ',') { c = fgetc(f); continue; }
    int len = 0;
    while (c != EOF && c != ' ' && c != '\t' && c != '\r' && c != '\n' && c != '#' && c != ',') {
      if (len < (int)sizeof(buf) - 1) buf[len++] = (char)c;
      else { fclose(f); return set_error(ATX_EINVAL, "%s:%d: token too long", path, lineno); }
      c = fgetc(f);
    }
    buf[len] = 0;
    char* end = nullptr;
    const double v = strtod(buf, &end);
    if (end == buf || *end != 0) {
      fclose(f);
      return set_error(ATX_EINVAL, "%s:%d: cannot parse '%s' as a number", path, lineno, buf);
    }
    if (integral && (v != floor(v) || fabs(v) > 2147483647.0)) {
      fclose(f);
      return set_error(ATX_EINVAL, "%s:%d: '%s' is not an integer", path, lineno, buf);
    }
    if (n >= capacity) {
      fclose(f);
      return set_error(ATX_ERANGE, "%s: more than %lld values", path, capacity);
    }
    out[n++] = (float)v;
  }
  fclose(f);
  *count = n;
  return ATX_OK;
}

int atx_lre_tables(const float* lut, int offset, float* grad_a, float* grad_b,
                   hipStream_t stream) {
  ATX_REQUIRE(lut && grad_a && grad_b, "atx_lre_tables: null pointer");
  ATX_REQUIRE(offset == 0 || offset == 128, "atx_lre_tables: offset must be 0 or 128");
  hipLaunchKernelGGL(lre_tables_kernel, dim3(2), dim3(256), 0, stream, lut, offset, grad_a,
                     grad_b);
  return check_launch("lre_tables_kernel");
}

int atx_date_tables(const float* lut, int half_ws, float* grad_a, float* grad_b,
                    hipStream_t stream) {
  ATX_REQUIRE(lut && grad_a && grad_b, "atx_date_tables: null pointer");
  ATX_REQUIRE(half_ws >= 0 && half_ws <= 127, "atx_date_tables: half_ws must be in [0, 127]");
  hipLaunchKernelGGL(date_tables_kernel, dim3(512), dim3(256), 0, stream, lut, half_ws, grad_a,
                     grad_b);
  return check_launch("date_tables_kernel");
}

}  // extern "C"
