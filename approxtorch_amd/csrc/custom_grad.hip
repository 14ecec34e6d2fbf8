// Custom (pair-wise 256x256 table) gradients of the LUT GEMM:
//   grad_x[n,k,l] = sum_o dy[n,o,l] * dx_lut[xi(n,k,l)*256 + wi(o,k)]   (ascending o)
//   grad_w[o,k]   = sum_{n,l} dy[n,o,l] * dw_lut[xi(n,k,l)*256 + wi(o,k)]
// Reference: csrc/cuda/bgemm_custom_grad_optimize.cu:30-116 and 136-205
// (uint8 indices), 315-404 and 419-490 (int8 values, index v+128).
//
// The fp32 tables are 256 KiB each (more than the 160 KiB LDS), so entries
// are gathered through the L1/L2 caches; dy and the index tiles are staged in
// LDS.  grad_w splits the (n,l) contraction across workgroups and reduces the
// partial sums in a second kernel.

#include "atx_internal.h"

#include <algorithm>

namespace atx {

constexpr int DX_L = 64, DX_K = 4, DX_O = 64;      // grad_x block tile
constexpr int DW_O = 16, DW_K = 16, DW_P = 64;     // grad_w block tile

template <bool SIGNED>
__device__ __forceinline__ unsigned idx_of(const void* base, long long i) {
  if (SIGNED) return (unsigned)((int)((const int8_t*)base)[i] + 128);
  return (unsigned)((const uint8_t*)base)[i];
}

template <bool SIGNED>
__global__ void __launch_bounds__(DX_L * DX_K)
custom_dx_kernel(const void* __restrict__ x, const void* __restrict__ w,
                 const float* __restrict__ dy, const float* __restrict__ lut, int K, int L,
                 int O, float* __restrict__ gx) {
  __shared__ float sdy[DX_O][DX_L];
  __shared__ unsigned short sw[DX_O][DX_K];
  const int n = blockIdx.z;
  const int k0 = blockIdx.y * DX_K, l0 = blockIdx.x * DX_L;
  const int tl = threadIdx.x % DX_L, tk = threadIdx.x / DX_L;
  const int l = l0 + tl, k = k0 + tk;
  const bool valid = l < L && k < K;
  const unsigned row = valid ? idx_of<SIGNED>(x, ((long long)n * K + k) * L + l) * 256u : 0u;
  float acc = 0.0f;
  for (int ob = 0; ob < O; ob += DX_O) {
    for (int i = threadIdx.x; i < DX_O * DX_L; i += DX_L * DX_K) {
      const int oo = i / DX_L, ll = i % DX_L;
      const int o = ob + oo, lg = l0 + ll;
      sdy[oo][ll] = (o < O && lg < L) ? dy[((long long)n * O + o) * L + lg] : 0.0f;
    }
    for (int i = threadIdx.x; i < DX_O * DX_K; i += DX_L * DX_K) {
      const int oo = i / DX_K, kk = i % DX_K;
      const int o = ob + oo, kg = k0 + kk;
      sw[oo][kk] = (o < O && kg < K) ? (unsigned short)idx_of<SIGNED>(w, (long long)o * K + kg)
                                     : (unsigned short)0;
    }
    __syncthreads();
    if (valid) {
      const int oe = min(DX_O, O - ob);
      // fused multiply-add, as the reference's contracted acc += dy * lut
      for (int oo = 0; oo < oe; ++oo) acc = fmaf(sdy[oo][tl], lut[row + sw[oo][tk]], acc);
    }
    __syncthreads();
  }
  if (valid) gx[((long long)n * K + k) * L + l] = acc;
}

// Partial grad_w over the p-range of split s: ws[s][o][k].
template <bool SIGNED>
__global__ void __launch_bounds__(DW_O * DW_K)
custom_dw_kernel(const void* __restrict__ x, const void* __restrict__ w,
                 const float* __restrict__ dy, const float* __restrict__ lut, int K, int L,
                 int O, long long P, long long p_chunk, float* __restrict__ ws) {
  __shared__ float sdy[DW_P][DW_O];
  __shared__ unsigned short sx[DW_P][DW_K];
  const int o0 = blockIdx.y * DW_O, k0 = blockIdx.x * DW_K;
  const int to = threadIdx.x / DW_K, tk = threadIdx.x % DW_K;
  const int o = o0 + to, k = k0 + tk;
  const bool valid = o < O && k < K;
  const unsigned col = valid ? idx_of<SIGNED>(w, (long long)o * K + k) : 0u;
  const long long pb = blockIdx.z * p_chunk;
  const long long pe = std::min<long long>(P, pb + p_chunk);
  float acc = 0.0f;
  for (long long p0 = pb; p0 < pe; p0 += DW_P) {
    for (int i = threadIdx.x; i < DW_P * DW_O; i += DW_O * DW_K) {
      const int pp = i % DW_P, oo = i / DW_P;
      const long long p = p0 + pp;
      float v = 0.0f;
      if (p < pe && o0 + oo < O) {
        const long long nn = p / L, ll = p - nn * L;
        v = dy[(nn * O + o0 + oo) * L + ll];
      }
      sdy[pp][oo] = v;
    }
    for (int i = threadIdx.x; i < DW_P * DW_K; i += DW_O * DW_K) {
      const int pp = i % DW_P, kk = i / DW_P;
      const long long p = p0 + pp;
      unsigned v = 0;
      if (p < pe && k0 + kk < K) {
        const long long nn = p / L, ll = p - nn * L;
        v = idx_of<SIGNED>(x, (nn * K + k0 + kk) * L + ll);
      }
      sx[pp][kk] = (unsigned short)v;
    }
    __syncthreads();
    if (valid) {
      const int pn = (int)std::min<long long>(DW_P, pe - p0);
      for (int pp = 0; pp < pn; ++pp)
        acc = fmaf(sdy[pp][to], lut[sx[pp][tk] * 256u + col], acc);
    }
    __syncthreads();
  }
  if (valid) ws[(long long)blockIdx.z * O * K + (long long)o * K + k] = acc;
}

__global__ void custom_split_sum_kernel(const float* __restrict__ ws, int S, long long numel,
                                        float* __restrict__ out) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < numel; i += stride) {
    float a = 0.0f;
    for (int s = 0; s < S; ++s) a += ws[(long long)s * numel + i];
    out[i] = a;
  }
}

static int dw_splits(int O, int K, long long P) {
  const long long tiles = cdiv(O, DW_O) * cdiv(K, DW_K);
  long long s = 1;
  while (tiles * s < 2048 && P / (s * 2) >= 4 * DW_P) s *= 2;
  return (int)s;
}

}  // namespace atx

using namespace atx;

extern "C" {

int atx_custom_grad_dx(const void* x, const void* w, int is_signed, const float* dy,
                       const float* dx_lut, int N, int K, int L, int O, float* grad_x,
                       hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0 && O >= 0, "atx_custom_grad_dx: negative size");
  if ((long long)N * K * L == 0) return ATX_OK;
  ATX_REQUIRE(x && dx_lut && grad_x && (O == 0 || (w && dy)), "atx_custom_grad_dx: null");
  ATX_REQUIRE(N <= 65535 && cdiv(K, DX_K) <= 65535, "atx_custom_grad_dx: grid too large");
  dim3 grid((unsigned)cdiv(L, DX_L), (unsigned)cdiv(K, DX_K), (unsigned)N);
  if (is_signed)
    hipLaunchKernelGGL(custom_dx_kernel<true>, grid, dim3(DX_L * DX_K), 0, stream, x, w, dy,
                       dx_lut, K, L, O, grad_x);
  else
    hipLaunchKernelGGL(custom_dx_kernel<false>, grid, dim3(DX_L * DX_K), 0, stream, x, w, dy,
                       dx_lut, K, L, O, grad_x);
  return check_launch("custom_dx_kernel");
}

long long atx_custom_grad_dw_workspace_bytes(int N, int K, int L, int O) {
  if (N <= 0 || K <= 0 || L <= 0 || O <= 0) return 0;
  return (long long)dw_splits(O, K, (long long)N * L) * O * K * 4;
}

int atx_custom_grad_dw(const void* x, const void* w, int is_signed, const float* dy,
                       const float* dw_lut, int N, int K, int L, int O, float* grad_w,
                       float* workspace, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0 && O >= 0, "atx_custom_grad_dw: negative size");
  const long long numel = (long long)O * K;
  if (numel == 0) return ATX_OK;
  ATX_REQUIRE(w && dw_lut && grad_w, "atx_custom_grad_dw: null pointer");
  const long long P = (long long)N * L;
  if (P == 0) {
    hipLaunchKernelGGL(custom_split_sum_kernel, dim3(elem_grid(numel, 256)), dim3(256), 0,
                       stream, (const float*)nullptr, 0, numel, grad_w);
    return check_launch("custom_split_sum_kernel");
  }
  ATX_REQUIRE(x && dy && workspace, "atx_custom_grad_dw: null operand/workspace");
  const int S = dw_splits(O, K, P);
  const long long chunk = cdiv(cdiv(P, S), DW_P) * DW_P;
  const int Sreal = (int)cdiv(P, chunk);
  dim3 grid((unsigned)cdiv(K, DW_K), (unsigned)cdiv(O, DW_O), (unsigned)Sreal);
  if (is_signed)
    hipLaunchKernelGGL(custom_dw_kernel<true>, grid, dim3(DW_O * DW_K), 0, stream, x, w, dy,
                       dw_lut, K, L, O, P, chunk, workspace);
  else
    hipLaunchKernelGGL(custom_dw_kernel<false>, grid, dim3(DW_O * DW_K), 0, stream, x, w, dy,
                       dw_lut, K, L, O, P, chunk, workspace);
  int rc = check_launch("custom_dw_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(custom_split_sum_kernel, dim3(elem_grid(numel, 256)), dim3(256), 0, stream,
                     workspace, Sreal, numel, grad_w);
  return check_launch("custom_split_sum_kernel");
}

}  // extern "C"
