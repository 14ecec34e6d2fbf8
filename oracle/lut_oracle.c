/*
 * CPU oracle for the LUT GEMM — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline load it,
 * and only as the checker; the product path never calls it.
 *
 * Restates the sum the reference computes in
 *   csrc/naive_cuda/bgemm_naive.cu:32-58   (one output per thread, int32 sum)
 *   csrc/claude/bgemm_lut_kernels.cuh:276-284 (fp32 sum in ascending k)
 * y[n,o,l] = sum_k lut[xi[n,k,l] * 256 + wi[o,k]]  (xi, wi: uint8 LUT indices)
 */
#include <stdint.h>

/* Exact int64 sum (lut holds integer values as int64). */
void oracle_lut_gemm_i64(const uint8_t* xi, const uint8_t* wi, const int64_t* lut,
                         int N, int K, int L, int O, int64_t* y) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int o = 0; o < O; ++o) {
      const uint8_t* w = wi + (long long)o * K;
      int64_t* yo = y + ((long long)n * O + o) * L;
      for (int l = 0; l < L; ++l) yo[l] = 0;
      for (int k = 0; k < K; ++k) {
        const int64_t* row_w = lut + w[k];            /* column w[k] of the LUT */
        const uint8_t* x = xi + ((long long)n * K + k) * L;
        for (int l = 0; l < L; ++l) yo[l] += row_w[(int)x[l] << 8];
      }
    }
}

/* fp32 sum in ascending k with plain (non-fused) adds: the reference's
 * non-split-K accumulation order. */
void oracle_lut_gemm_f32(const uint8_t* xi, const uint8_t* wi, const float* lut, int N,
                         int K, int L, int O, float* y) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int o = 0; o < O; ++o) {
      const uint8_t* w = wi + (long long)o * K;
      float* yo = y + ((long long)n * O + o) * L;
      for (int l = 0; l < L; ++l) yo[l] = 0.0f;
      for (int k = 0; k < K; ++k) {
        const float* row_w = lut + w[k];
        const uint8_t* x = xi + ((long long)n * K + k) * L;
        for (int l = 0; l < L; ++l) {
          volatile float t = yo[l] + row_w[(int)x[l] << 8];
          yo[l] = t;
        }
      }
    }
}

/* Pair-table ("custom" estimator) gradients of the LUT GEMM in fp64:
 *   gx[n,k,l] = sum_o go[n,o,l] * dx[xi[n,k,l] * 256 + wi[o,k]]   (ascending o)
 *   gw[o,k]   = sum_{n,l} go[n,o,l] * dw[xi[n,k,l] * 256 + wi[o,k]]
 * csrc/naive_cuda/bgemm_custom_grad_naive.cu:28-92 (one output per thread). */
void oracle_custom_grads_f64(const uint8_t* xi, const uint8_t* wi, const double* go,
                             const double* dx, const double* dw, int N, int K, int L, int O,
                             double* gx, double* gw) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) {
      const uint8_t* x = xi + ((long long)n * K + k) * L;
      double* g = gx + ((long long)n * K + k) * L;
      for (int l = 0; l < L; ++l) g[l] = 0.0;
      for (int o = 0; o < O; ++o) {
        const double* col = dx + wi[(long long)o * K + k];
        const double* gr = go + ((long long)n * O + o) * L;
        for (int l = 0; l < L; ++l) g[l] += gr[l] * col[(int)x[l] << 8];
      }
    }
#pragma omp parallel for collapse(2) schedule(static)
  for (int o = 0; o < O; ++o)
    for (int k = 0; k < K; ++k) {
      const double* col = dw + wi[(long long)o * K + k];
      double s = 0.0;
      for (int n = 0; n < N; ++n) {
        const uint8_t* x = xi + ((long long)n * K + k) * L;
        const double* gr = go + ((long long)n * O + o) * L;
        for (int l = 0; l < L; ++l) s += gr[l] * col[(int)x[l] << 8];
      }
      gw[(long long)o * K + k] = s;
    }
}
