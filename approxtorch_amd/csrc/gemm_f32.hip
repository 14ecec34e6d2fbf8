// fp32 matrix-core (MFMA) GEMMs for the STE / LRE backward of the LUT conv.
//
// Both estimators differentiate y[n,o,l] = sum_k f(x_nkl, w_ok) as a dense
// product of mapped operands (STE: the quantized values, LRE: 256-entry slope
// tables indexed by the other operand's LUT index):
//   col[n,k,l] = sum_o go[n,o,l] * Tx[wi(o,k)]          (backward-data, then fold)
//   gw[o,k]    = sum_{n,l} go[n,o,l] * Tw[xi(n,k,l)]     (backward-weight)
// with xi read straight from the saved quantized image (implicit im2col;
// out-of-image taps take index pad_index, so LRE's Tw[128] border rule
// holds).  Reference: csrc/claude/bgemm_lre_backward_claude.cu:443-524 (cuBLAS
// SGEMMs) and nn/bgemm_int8.py:184-207,277-290 (cuDNN convolution_backward).
//
// Kernel: 128x128 block tile, 16-deep k-tile, 256 threads (2x2 waves of
// 64x64, each 2x2 v_mfma_f32_32x32x2f32), double-buffered LDS tiles fed by
// register prefetch.  gfx950 has no reduced-precision fp32 mode, so results
// are plain fp32 products with fp32 accumulation.

#include "atx_internal.h"

#include <algorithm>

namespace atx {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int GT = 256;
constexpr int LDA = BM + 4, LDB = BN + 4;   // padded LDS rows (bank spread)

// Loader for the data-gradient GEMM, batch n = blockIdx.z:
//   A(m = k, p = o) = Tx[wq[o*K + k]],  B(p = o, j = l) = go[n][o][l].
struct DataOperands {
  const uint8_t* wq; const float* go; const float* tx;
  int K, O, L;
  __device__ float a(int m, int p, int) const {
    return (m < K && p < O) ? tx[wq[(long long)p * K + m]] : 0.0f;
  }
  __device__ float b(int p, int j, int n) const {
    return (p < O && j < L) ? go[((long long)n * O + p) * L + j] : 0.0f;
  }
};

// Loader for the weight-gradient GEMM (p = n*L + l):
//   A(m = o, p) = go[n][o][l],  B(p, j = k) = Tw[index of image tap k at l].
template <typename T>
struct WeightOperands {
  const float* go; const T* img; const float* tw; const float* pad_dev;
  atx_conv_geom g; int O, K, L, P, offset, pad_index;
  __device__ float a(int m, int p, int) const {
    if (m >= O || p >= P) return 0.0f;
    const int n = p / L, l = p - (p / L) * L;
    return go[((long long)n * O + m) * L + l];
  }
  __device__ float b(int p, int j, int) const {
    if (p >= P || j >= K) return 0.0f;
    const int n = p / L, l = p - (p / L) * L;
    const int KK = g.KH * g.KW;
    const int c = j / KK, t = j - (j / KK) * KK;
    const int kh = t / g.KW, kw = t - (t / g.KW) * g.KW;
    const int oh = l / g.OW, ow = l - (l / g.OW) * g.OW;
    const int ih = oh * g.SH + kh * g.DH - g.PH;
    const int iw = ow * g.SW + kw * g.DW - g.PW;
    unsigned v = pad_dev ? quant_index(pad_dev[0], 0) : (unsigned)pad_index;
    if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W) {
      const T x = img[(((long long)n * g.C + c) * g.H + ih) * g.W + iw];
      if constexpr (sizeof(T) == 4) v = quant_index((float)x, offset);
      else if constexpr (std::is_same<T, int8_t>::value) v = (unsigned)((int)x + 128);
      else v = (unsigned)x;
    }
    return tw[v];
  }
};

// Thread -> element maps for the tile loads.  The A tile is stored [p][m],
// B as [p][j].  `m_fast`: consecutive threads walk m (else p) for coalescing.
template <bool M_FAST>
__device__ __forceinline__ void tile_coord(int t, int i, int& p, int& m) {
  const int e = t + i * GT;                 // 0 .. BM*BK-1
  if (M_FAST) { m = e % BM; p = e / BM; }
  else { p = e % BK; m = e / BK; }
}

template <typename OPS, bool A_M_FAST, bool B_J_FAST>
__global__ void __launch_bounds__(GT, 2)
mfma_gemm_kernel(OPS ops, int M, int N, int P, int p_chunk, float* __restrict__ out,
                 long long out_bstride, long long out_sstride) {
  __shared__ float As[2][BK][LDA];
  __shared__ float Bs[2][BK][LDB];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int zb = blockIdx.z;
  // grid.z enumerates (batch, split): z = batch * S + s
  const int S = (P + p_chunk - 1) / p_chunk;
  const int batch = zb / S, s = zb % S;
  const int pb = s * p_chunk, pe = min(P, pb + p_chunk);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  constexpr int PER = BM * BK / GT;   // 8 elements per thread per tile
  float ra[PER], rb[PER];
  auto fetch = [&](int p0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int p, m;
      tile_coord<A_M_FAST>(t, i, p, m);
      const int gp = p0 + p;
      ra[i] = (gp < pe) ? ops.a(m0 + m, gp, batch) : 0.0f;
      int pj, j;
      tile_coord<B_J_FAST>(t, i, pj, j);
      const int gpj = p0 + pj;
      rb[i] = (gpj < pe) ? ops.b(gpj, n0 + j, batch) : 0.0f;
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int p, m;
      tile_coord<A_M_FAST>(t, i, p, m);
      As[buf][p][m] = ra[i];
      int pj, j;
      tile_coord<B_J_FAST>(t, i, pj, j);
      Bs[buf][pj][j] = rb[i];
    }
  };

  if (pb < pe) {
    fetch(pb);
    stash(0);
    __syncthreads();
    int buf = 0;
    for (int p0 = pb; p0 < pe; p0 += BK) {
      const bool more = p0 + BK < pe;
      if (more) fetch(p0 + BK);
#pragma unroll
      for (int kk = 0; kk < BK; kk += 2) {
        const int kr = kk + (lane >> 5);
        float av[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) av[i] = As[buf][kr][wm * 64 + i * 32 + (lane & 31)];
#pragma unroll
        for (int j = 0; j < 2; ++j) bv[j] = Bs[buf][kr][wn * 64 + j * 32 + (lane & 31)];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
      if (more) stash(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  }

  // D layout of 32x32x2: lane holds rows 8*(r/4) + 4*(lane/32) + r%4, col lane%32.
  float* o = out + (long long)batch * out_bstride + (long long)s * out_sstride;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int col = n0 + wn * 64 + j * 32 + (lane & 31);
        if (row < M && col < N) o[(long long)row * N + col] = acc[i][j][r];
      }
}

// gw[i] = sum_s ws[s][i]; optional fused per-channel fake-quant backward:
// gw = mask ? sum / max(scale[o], 1e-12) : 0 with o = i / K.
__global__ void split_sum_kernel(const float* __restrict__ ws, int S, long long numel, int K,
                                 const uint8_t* __restrict__ mask,
                                 const float* __restrict__ scale, float* __restrict__ out) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < numel; i += stride) {
    float a = 0.0f;
    for (int s = 0; s < S; ++s) a += ws[(long long)s * numel + i];
    if (mask) a = (mask[i] ? a : 0.0f) / fmaxf(scale[i / K], 1e-12f);
    out[i] = a;
  }
}

// Split of the weight-gradient contraction: enough blocks to fill 256 CUs.
static int weight_splits(int M, int N, long long P) {
  const long long tiles = cdiv(M, BM) * cdiv(N, BN);
  long long s = 1;
  while (tiles * s < 1024 && P / (s * 2) >= 4 * BK) s *= 2;
  return (int)s;
}

}  // namespace atx

using namespace atx;

extern "C" {

int atx_conv_bwd_data_col(const float* go, const uint8_t* wq, const float* tx, int N, int O,
                          int K, int L, float* col, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && O >= 0 && K >= 0 && L >= 0, "atx_conv_bwd_data_col: negative size");
  if ((long long)N * K * L == 0) return ATX_OK;
  ATX_REQUIRE(col, "atx_conv_bwd_data_col: null output");
  if (O == 0) {
    // Empty contraction: the split-sum kernel with S = 0 writes zeros.
    const long long numel = (long long)N * K * L;
    hipLaunchKernelGGL(split_sum_kernel, dim3(elem_grid(numel, 256)), dim3(256), 0, stream,
                       (const float*)nullptr, 0, numel, K, (const uint8_t*)nullptr,
                       (const float*)nullptr, col);
    return check_launch("split_sum_kernel");
  }
  ATX_REQUIRE(go && wq && tx, "atx_conv_bwd_data_col: null pointer");
  ATX_REQUIRE(N <= 65535, "atx_conv_bwd_data_col: batch too large");
  DataOperands ops{wq, go, tx, K, O, L};
  dim3 grid((unsigned)cdiv(L, BN), (unsigned)cdiv(K, BM), (unsigned)N);
  hipLaunchKernelGGL((mfma_gemm_kernel<DataOperands, true, true>), grid, dim3(GT), 0, stream,
                     ops, K, L, O, O > 0 ? O : 1, col, (long long)K * L, 0LL);
  return check_launch("mfma_gemm_kernel<data>");
}

long long atx_conv_bwd_weight_workspace_bytes(int O, int K, long long P) {
  if (O <= 0 || K <= 0 || P <= 0) return 0;
  return (long long)weight_splits(O, K, P) * O * K * 4;
}

int atx_conv_bwd_weight(const float* go, const void* img, int dtype, atx_conv_geom g, int O,
                        int pad_index, const float* pad_dev, const float* tw,
                        const uint8_t* mask_w, const float* scale_w, float* gw,
                        float* workspace, hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && dtype >= 0 && dtype <= 3, "atx_conv_bwd_weight: bad arguments");
  const int f32_offset = dtype == 3 ? 0 : 128;   // 3: fp32 unsigned quantized values
  if (dtype == 3) dtype = 2;
  ATX_REQUIRE(pad_index >= 0 && pad_index <= 255, "atx_conv_bwd_weight: bad pad_index");
  const int K = g.C * g.KH * g.KW;
  const int L = g.OH * g.OW;
  const long long P = (long long)g.N * L;
  ATX_REQUIRE(P < 0x7fffffffLL, "atx_conv_bwd_weight: N*L too large");
  if ((long long)O * K == 0) return ATX_OK;
  ATX_REQUIRE(gw && tw && (!mask_w || scale_w), "atx_conv_bwd_weight: null pointer");
  if (P == 0) {
    // Empty contraction: the split-sum kernel with S = 0 writes zeros.
    hipLaunchKernelGGL(split_sum_kernel, dim3(elem_grid((long long)O * K, 256)), dim3(256), 0,
                       stream, (const float*)nullptr, 0, (long long)O * K, K,
                       (const uint8_t*)nullptr, scale_w, gw);
    return check_launch("split_sum_kernel");
  }
  ATX_REQUIRE(go && img && workspace, "atx_conv_bwd_weight: null operand/workspace");
  const int S = weight_splits(O, K, P);
  const int chunk = (int)(cdiv(cdiv(P, S), BK) * BK);
  const int Sreal = (int)cdiv(P, chunk);
  dim3 grid((unsigned)cdiv(K, BN), (unsigned)cdiv(O, BM), (unsigned)Sreal);
  const long long sst = (long long)O * K;
  if (dtype == 0) {
    WeightOperands<int8_t> ops{go, (const int8_t*)img, tw, pad_dev, g, O, K, L, (int)P, 128,
                               pad_index};
    hipLaunchKernelGGL((mfma_gemm_kernel<WeightOperands<int8_t>, false, false>), grid, dim3(GT),
                       0, stream, ops, O, K, (int)P, chunk, workspace, 0LL, sst);
  } else if (dtype == 1) {
    WeightOperands<uint8_t> ops{go, (const uint8_t*)img, tw, pad_dev, g, O, K, L, (int)P, 0,
                                pad_index};
    hipLaunchKernelGGL((mfma_gemm_kernel<WeightOperands<uint8_t>, false, false>), grid,
                       dim3(GT), 0, stream, ops, O, K, (int)P, chunk, workspace, 0LL, sst);
  } else {
    WeightOperands<float> ops{go, (const float*)img, tw, pad_dev, g, O, K, L, (int)P,
                              f32_offset, pad_index};
    hipLaunchKernelGGL((mfma_gemm_kernel<WeightOperands<float>, false, false>), grid, dim3(GT),
                       0, stream, ops, O, K, (int)P, chunk, workspace, 0LL, sst);
  }
  int rc = check_launch("mfma_gemm_kernel<weight>");
  if (rc) return rc;
  hipLaunchKernelGGL(split_sum_kernel, dim3(elem_grid(sst, 256)), dim3(256), 0, stream,
                     workspace, Sreal, sst, K, mask_w, scale_w, gw);
  return check_launch("split_sum_kernel");
}

}  // extern "C"
