// Depthwise LUT conv (groups == C == O, one filter per channel) and its STE /
// LRE backward.
//
//   y[n,c,oh,ow] = sum_{i,j} LUT[xi(n, c, oh*SH - PH + i*DH, ow*SW - PW + j*DW)][wi(c, i, j)]
//
// Out-of-image taps take LUT row pad_index (128 = quantized zero of int8),
// as the im2col pipeline's zero padding does.  Reference:
// csrc/claude/dwconv_claude.cu:1-285 (forward) and the grouped
// convolution_backward of nn/bgemm_int8.py:162-212,259-295.
//
// Forward: a block owns a run of one channel's N*OH*OW outputs; the channel's
// KH*KW table columns LUT[.][wi(c,t)] (512 B each in the 16-bit image) are
// staged in LDS, every thread walks output pixels and sums its taps in
// ascending (i, j) order: exact int32 for the integer LUT classes, fp32 in
// the same order for the fp32 fallback (bit-identical to a per-channel LUT
// GEMM).  The work is small next to the dense convs (K = KH*KW per output),
// so the kernel is bound by the image and output traffic.
//
// Backward (per channel, tables indexed by the other operand):
//   gx[n,c,h,w] = sum over taps (i,j) and outputs (oh,ow) reading (h,w) of
//                 go'[n,c,oh,ow] * tx[wi(c,i,j)]
//   gw[c,i,j]   = sum_{n,oh,ow} go'[n,c,oh,ow] * tw[xi(n,c,tap)]
// with go' = go * fp32(sx * sw[c]) when a go scale is given, and the
// fake-quant STE masks fused into the outputs.

#include "atx_internal.h"
#include "atx_tiles.h"

#include <algorithm>
#include <type_traits>

namespace atx {

constexpr int DW_THREADS = 256;
constexpr int DW_MAX_TAPS = 64;         // LDS: 64 taps x 256 entries x 4 B = 64 KiB
constexpr int DW_WSPLIT_ROWS = 4096;    // contraction rows per weight-gradient block
#ifndef DW_STRIP_GROUP
#define DW_STRIP_GROUP 2                // strips per in-flight group of the 3x3 strip kernel
#endif

template <typename T> __device__ __forceinline__ unsigned dw_index(T v, int offset);
template <> __device__ __forceinline__ unsigned dw_index<int8_t>(int8_t v, int) {
  return (unsigned)((int)v + 128);
}
template <> __device__ __forceinline__ unsigned dw_index<uint8_t>(uint8_t v, int) {
  return (unsigned)v;
}
template <> __device__ __forceinline__ unsigned dw_index<float>(float v, int offset) {
  return quant_index(v, offset);
}

struct DwEpilogue {
  int out_kind; const float* sx; const float* sw; const float* bias;
};

// Stages the channel's KK table columns tab[t][x] = LUT[x][wi(c, t)]
// (DW_THREADS == 256 threads, thread = x), eight taps' loads in flight at a
// time, then a barrier.  wc = the channel's KK weight indices.
template <typename ENTRY, bool SIGNED>
__device__ __forceinline__ void stage_tables(ENTRY* tab, const uint8_t* __restrict__ wc, int KK,
                                             const uint16_t* __restrict__ lut16t,
                                             const float* __restrict__ lutf32t) {
  static_assert(DW_THREADS == 256, "one thread per table entry");
  const unsigned x = threadIdx.x;
  for (int t0 = 0; t0 < KK; t0 += 8) {
    ENTRY v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (t0 + u < KK) {
        const unsigned w = wc[t0 + u];
        if constexpr (sizeof(ENTRY) == 4 && !std::is_integral<ENTRY>::value) {
          v[u] = lutf32t[w * 256u + x];
        } else {
          const unsigned e = lut16t[w * 256u + x];
          v[u] = SIGNED ? (int)(short)(unsigned short)e : (int)e;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (t0 + u < KK) tab[(t0 + u) * 256 + x] = v[u];
  }
  __syncthreads();
}

// ENTRY: int (16-bit classes, sign-extended or not) or float (fp32 class).
template <typename T, typename ENTRY, bool SIGNED>
__global__ void __launch_bounds__(DW_THREADS)
dwconv_fwd_kernel(const T* __restrict__ img, atx_conv_geom g, int offset, int pad,
                  const uint8_t* __restrict__ wq, const uint16_t* __restrict__ lut16t,
                  const float* __restrict__ lutf32t, DwEpilogue ep, void* __restrict__ y,
                  int chunk) {
  extern __shared__ __align__(16) unsigned char dw_smem[];
  ENTRY* tab = (ENTRY*)dw_smem;
  const int c = blockIdx.y;
  const int KK = g.KH * g.KW;
  stage_tables<ENTRY, SIGNED>(tab, wq + (long long)c * KK, KK, lut16t, lutf32t);
  const int L = g.OH * g.OW;
  float sc = 1.0f, bi = 0.0f;
  if (ep.out_kind == ATX_OUT_DEQUANT) {
    sc = ep.sx[0] * ep.sw[c];
    if (ep.bias) bi = ep.bias[c];
  }
  // this block's run of the channel's N*L outputs (p = n*L + l)
  const long long P = (long long)g.N * L;
  const long long pb = (long long)blockIdx.x * chunk;
  const long long pe = min(P, pb + chunk);
  for (long long p = pb + threadIdx.x; p < pe; p += blockDim.x) {
    const int n = (int)(p / L), l = (int)(p - (long long)n * L);
    const T* plane = img + ((long long)n * g.C + c) * g.H * g.W;
    const long long ybase = ((long long)n * g.C + c) * L;
    const int oh = l / g.OW, ow = l - oh * g.OW;
    ENTRY acc = 0;
    for (int i = 0; i < g.KH; ++i) {
      const int ih = oh * g.SH - g.PH + i * g.DH;
      const bool hin = (unsigned)ih < (unsigned)g.H;
      for (int j = 0; j < g.KW; ++j) {
        const int iw = ow * g.SW - g.PW + j * g.DW;
        unsigned xi = (unsigned)pad;
        if (hin && (unsigned)iw < (unsigned)g.W) xi = dw_index<T>(plane[ih * g.W + iw], offset);
        acc += tab[(i * g.KW + j) * 256 + xi];
      }
    }
    if (ep.out_kind == ATX_OUT_I32) {
      ((int*)y)[ybase + l] = (int)acc;
    } else if (ep.out_kind == ATX_OUT_DEQUANT) {
      const float t = (float)acc * sc;
      ((float*)y)[ybase + l] = ep.bias ? bi + t : t;
    } else {
      ((float*)y)[ybase + l] = (float)acc;
    }
  }
}

// Stores a strip's four sums acc[] at output element ybase (int32, fp32, or
// dequantized fp32 sc * acc + bi); `left` = outputs left in the row (only
// min(4, left) are stored).  vec: one 16-byte store (the caller guarantees
// OW % 4 == 0 and a 16-byte aligned y).
template <typename ENTRY>
__device__ __forceinline__ void store_strip(const ENTRY (&acc)[4], const DwEpilogue& ep,
                                            float sc, float bi, void* __restrict__ y,
                                            long long ybase, int left, bool vec) {
  if (ep.out_kind == ATX_OUT_I32) {
    int* yo = (int*)y + ybase;
    if (vec) {
      *(int4*)yo = make_int4((int)acc[0], (int)acc[1], (int)acc[2], (int)acc[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < left) yo[e] = (int)acc[e];
    }
    return;
  }
  float f[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (ep.out_kind == ATX_OUT_DEQUANT) {
      const float t = (float)acc[e] * sc;
      f[e] = ep.bias ? bi + t : t;
    } else {
      f[e] = (float)acc[e];
    }
  }
  float* yo = (float*)y + ybase;
  if (vec) {
    *(float4*)yo = make_float4(f[0], f[1], f[2], f[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < left) yo[e] = f[e];
  }
}

// Strip form of dwconv_fwd_kernel for KW == 3, dilation 1 along W, stride
// SW (1 or 2) along W: a thread owns four consecutive outputs of one output
// row (a strip; strips index (n, oh, quad of ow) of the channel), decomposes
// its index once, and per kernel row reads the 3 + 4*SW - SW input values
// its four outputs need once (6 for SW = 1, 9 for SW = 2), then sums each
// output's taps in the same ascending (i, j) order as dwconv_fwd_kernel
// (identical results).  With OW % 4 == 0 the strip is stored as one 16-byte
// vector (`vec`: OW % 4 == 0 and y 16-byte aligned).
template <typename T, typename ENTRY, bool SIGNED, int SW>
__global__ void __launch_bounds__(DW_THREADS)
dwconv_fwd_strip_kernel(const T* __restrict__ img, atx_conv_geom g, int offset, int pad,
                        const uint8_t* __restrict__ wq, const uint16_t* __restrict__ lut16t,
                        const float* __restrict__ lutf32t, DwEpilogue ep, void* __restrict__ y,
                        int chunk, bool vec) {
  constexpr int NX = 3 * SW + 3;           // input columns of a strip (SW*3 + 3)
  extern __shared__ __align__(16) unsigned char dw_smem[];
  ENTRY* tab = (ENTRY*)dw_smem;
  const int c = blockIdx.y;
  const int KK = g.KH * 3;
  stage_tables<ENTRY, SIGNED>(tab, wq + (long long)c * KK, KK, lut16t, lutf32t);
  const int L = g.OH * g.OW;
  float sc = 1.0f, bi = 0.0f;
  if (ep.out_kind == ATX_OUT_DEQUANT) {
    sc = ep.sx[0] * ep.sw[c];
    if (ep.bias) bi = ep.bias[c];
  }
  const int Q = (g.OW + 3) >> 2;                 // strips per output row
  const int S = g.N * g.OH * Q;                  // strips of the channel
  const int sb = blockIdx.x * chunk, se = min(S, sb + chunk);
  for (int s = sb + (int)threadIdx.x; s < se; s += blockDim.x) {
    const int q = s % Q, r = s / Q;
    const int oh = r % g.OH, n = r / g.OH;
    const int ow0 = q << 2;
    const T* plane = img + ((long long)n * g.C + c) * g.H * g.W;
    const int iw0 = ow0 * SW - g.PW;             // first input column of the strip
    ENTRY acc[4] = {0, 0, 0, 0};
    for (int i = 0; i < g.KH; ++i) {
      const int ih = oh * g.SH - g.PH + i * g.DH;
      const bool hin = (unsigned)ih < (unsigned)g.H;
      unsigned xi[NX];
#pragma unroll
      for (int m = 0; m < NX; ++m) {
        const int iw = iw0 + m;
        xi[m] = (hin && (unsigned)iw < (unsigned)g.W)
                    ? dw_index<T>(plane[(long long)ih * g.W + iw], offset) : (unsigned)pad;
      }
      const ENTRY* trow = tab + i * 3 * 256;
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[e] += trow[j * 256 + xi[e * SW + j]];
    }
    store_strip(acc, ep, sc, bi, y, ((long long)n * g.C + c) * L + (long long)oh * g.OW + ow0,
                g.OW - ow0, vec);
  }
}

// The strips of dwconv_fwd_strip_kernel for 3x3 kernels (any stride and
// dilation along H) over a byte image (int8 when INT8, else uint8) that is
// 4-byte aligned with a byte size that is a multiple of 4 and below 2^31:
// identical sums, but
//  - a strip row's NX columns lie in the three aligned dwords from the
//    dword holding its first column (shift sh = first byte & 3 <= 3,
//    sh + NX <= 12), read with buffer loads over the whole image, so a row
//    costs three loads for any W and padding up to 4 (out-of-image columns
//    take the pad index).  The three loads merge into one 12-byte access:
//    dwords of it past the image's end read 0, but one starting before the
//    image (the first plane's top-left strips, window start -4) would read
//    0 for all three, so such a window is read from byte 0 and moved up one
//    dword in registers;
//  - each thread keeps two groups of U strips in flight: the 3 x 3 dwords
//    of the next group's strips are requested before the current group is
//    summed, and the first group's before the tables are staged;
//  - strip positions (q, oh, n) advance by the block's stride incrementally
//    (one carry each) instead of by division.
template <int U>
struct StripGroup {
  unsigned d[U][3][3];   // [strip][kernel row][dword]
  int q[U], oh[U], n[U];
};

template <typename ENTRY, bool SIGNED, bool INT8, int SW, int U>
__global__ void __launch_bounds__(DW_THREADS)
dwconv_fwd_strip3_kernel(const uint8_t* __restrict__ img, atx_conv_geom g, int pad,
                         const uint8_t* __restrict__ wq, const uint16_t* __restrict__ lut16t,
                         const float* __restrict__ lutf32t, DwEpilogue ep,
                         void* __restrict__ y, int chunk, bool vec) {
  constexpr int NX = 3 * SW + 3;
  constexpr int D = DW_THREADS;
  extern __shared__ __align__(16) unsigned char dw_smem[];
  ENTRY* tab = (ENTRY*)dw_smem;
  const int c = blockIdx.y;
  const int L = g.OH * g.OW;
  const int Q = (g.OW + 3) >> 2;                 // strips per output row
  const int S = g.N * g.OH * Q;                  // strips of the channel
  const int sb = blockIdx.x * chunk, se = min(S, sb + chunk);
  const unsigned HW = (unsigned)g.H * (unsigned)g.W;
  const __amdgpu_buffer_rsrc_t imr = buffer_rsrc(img, (int)((long long)g.N * g.C * HW));
  // position of strip s = sb + threadIdx.x, and the per-step increments
  int s = sb + (int)threadIdx.x;
  int q = s % Q, oh = (s / Q) % g.OH, n = (s / Q) / g.OH;
  const int dq = D % Q, dr = D / Q, doh = dr % g.OH, dn = dr / g.OH;
  // first dword of kernel row i of a strip at (q, oh, n): unsigned
  // arithmetic (a strip before the image wraps to an offset past its end)
  auto row_byte = [&](int q_, int oh_, int n_, int i) -> unsigned {
    return ((unsigned)n_ * (unsigned)g.C + (unsigned)c) * HW +
           (unsigned)(oh_ * g.SH - g.PH + i * g.DH) * (unsigned)g.W +
           (unsigned)((q_ << 2) * SW - g.PW);
  };
  auto fetch = [&](StripGroup<U>& G) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      G.q[u] = q; G.oh[u] = oh; G.n[u] = n;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        unsigned a = row_byte(q, oh, n, i) & ~3u;
        a = (int)a < 0 ? 0u : a;
#pragma unroll
        for (int k = 0; k < 3; ++k)
          G.d[u][i][k] = __builtin_amdgcn_raw_buffer_load_b32(imr, (int)(a + 4u * k), 0, 0);
      }
      q += dq;
      const int cq = q >= Q;
      q -= cq ? Q : 0;
      oh += doh + cq;
      const int co = oh >= g.OH;
      oh -= co ? g.OH : 0;
      n += dn + co;
    }
  };
  StripGroup<U> cur, nxt;
  fetch(cur);
  stage_tables<ENTRY, SIGNED>(tab, wq + (long long)c * 9, 9, lut16t, lutf32t);
  float sc = 1.0f, bi = 0.0f;
  if (ep.out_kind == ATX_OUT_DEQUANT) {
    sc = ep.sx[0] * ep.sw[c];
    if (ep.bias) bi = ep.bias[c];
  }
  for (; s < se; s += U * D) {
    const bool more = s + U * D < se;
    if (more) fetch(nxt);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s + u * D >= se) break;
      const int q_ = cur.q[u], oh_ = cur.oh[u], n_ = cur.n[u];
      const int iw0 = (q_ << 2) * SW - g.PW;
      ENTRY acc[4] = {0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int ih = oh_ * g.SH - g.PH + i * g.DH;
        const bool hin = (unsigned)ih < (unsigned)g.H;
        const unsigned rb = row_byte(q_, oh_, n_, i), sh = rb & 3u;
        // the window's dwords (a window from byte -4 was read from byte 0)
        const bool early = (int)(rb & ~3u) < 0;
        const unsigned w0 = early ? 0u : cur.d[u][i][0];
        const unsigned w1 = early ? cur.d[u][i][0] : cur.d[u][i][1];
        const unsigned w2 = early ? cur.d[u][i][1] : cur.d[u][i][2];
        // columns 0..NX-1 of the row in bytes of e[0..2]
        unsigned e[3];
        e[0] = __builtin_amdgcn_alignbyte(w1, w0, sh);
        e[1] = __builtin_amdgcn_alignbyte(w2, w1, sh);
        e[2] = w2 >> (8u * sh);
        unsigned xi[NX];
#pragma unroll
        for (int m = 0; m < NX; ++m) {
          const unsigned b = (e[m >> 2] >> (8 * (m & 3))) & 255u;
          xi[m] = (hin && (unsigned)(iw0 + m) < (unsigned)g.W) ? (INT8 ? b ^ 128u : b)
                                                               : (unsigned)pad;
        }
        const ENTRY* trow = tab + i * 3 * 256;
#pragma unroll
        for (int o = 0; o < 4; ++o)
#pragma unroll
          for (int j = 0; j < 3; ++j) acc[o] += trow[j * 256 + xi[o * SW + j]];
      }
      store_strip(acc, ep, sc, bi, y,
                  ((long long)n_ * g.C + c) * L + (long long)oh_ * g.OW + (q_ << 2),
                  g.OW - (q_ << 2), vec);
    }
    if (more) cur = nxt;
  }
}

// gx for one image pixel: taps in ascending (i, j) order.
__global__ void __launch_bounds__(DW_THREADS)
dwconv_bwd_data_kernel(const float* __restrict__ go, const uint8_t* __restrict__ wq,
                       const float* __restrict__ tx, atx_conv_geom g,
                       const float* __restrict__ go_sx, const float* __restrict__ go_sw,
                       const uint8_t* __restrict__ mask, const float* __restrict__ scale,
                       float* __restrict__ gx) {
  __shared__ float stx[256];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) stx[i] = tx[i];
  __syncthreads();
  const int KK = g.KH * g.KW;
  const long long HW = (long long)g.H * g.W;
  const long long total = (long long)g.N * g.C * HW;
  const int L = g.OH * g.OW;
  const float sdiv = mask ? fmaxf(scale[0], 1e-12f) : 1.0f;
  for (long long e = blockIdx.x * (long long)blockDim.x + threadIdx.x; e < total;
       e += (long long)gridDim.x * blockDim.x) {
    const long long nc = e / HW;
    const int hw = (int)(e - nc * HW);
    const int h = hw / g.W, w = hw - (hw / g.W) * g.W;
    const int c = (int)(nc % g.C);
    const float s = go_sw ? go_sx[0] * go_sw[c] : 1.0f;
    const float* gp = go + nc * L;
    float a = 0.0f;
    for (int i = 0; i < g.KH; ++i) {
      const int th = h + g.PH - i * g.DH;
      if (th < 0 || th % g.SH) continue;
      const int oh = th / g.SH;
      if (oh >= g.OH) continue;
      for (int j = 0; j < g.KW; ++j) {
        const int tw_ = w + g.PW - j * g.DW;
        if (tw_ < 0 || tw_ % g.SW) continue;
        const int ow = tw_ / g.SW;
        if (ow >= g.OW) continue;
        const float gv = go_sw ? gp[oh * g.OW + ow] * s : gp[oh * g.OW + ow];
        a += gv * stx[wq[(long long)c * KK + i * g.KW + j]];
      }
    }
    if (mask) a = (mask[e] ? a : 0.0f) / sdiv;
    gx[e] = a;
  }
}

// Partial weight gradients: block (c, s) sums contraction rows
// [s*DW_WSPLIT_ROWS, ...) of P = N*OH*OW for every tap of channel c and
// writes ws[s][c][t].  Threads keep up to 16 taps at a time; the block
// reduction runs in a fixed order (deterministic).
template <typename T>
__global__ void __launch_bounds__(DW_THREADS)
dwconv_bwd_weight_kernel(const float* __restrict__ go, const T* __restrict__ img,
                         atx_conv_geom g, int offset, int pad, const float* __restrict__ pad_dev,
                         const float* __restrict__ tw, const float* __restrict__ go_sx,
                         const float* __restrict__ go_sw, float* __restrict__ ws) {
  __shared__ float stw[256];
  __shared__ float red[16][DW_THREADS + 1];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) stw[i] = tw[i];
  if (pad_dev) pad = (int)quant_index(pad_dev[0], 0);
  __syncthreads();
  const int c = blockIdx.x, s = blockIdx.y;
  const int KK = g.KH * g.KW;
  const int L = g.OH * g.OW;
  const long long P = (long long)g.N * L;
  const long long p0 = (long long)s * DW_WSPLIT_ROWS;
  const long long p1 = min(P, p0 + DW_WSPLIT_ROWS);
  const float sc = go_sw ? go_sx[0] * go_sw[c] : 1.0f;
  for (int t0 = 0; t0 < KK; t0 += 16) {
    float acc[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
    for (long long p = p0 + threadIdx.x; p < p1; p += blockDim.x) {
      const int n = (int)(p / L), l = (int)(p - (long long)n * L);
      const int oh = l / g.OW, ow = l - oh * g.OW;
      const float gv = go_sw ? go[((long long)n * g.C + c) * L + l] * sc
                             : go[((long long)n * g.C + c) * L + l];
      const T* plane = img + ((long long)n * g.C + c) * g.H * g.W;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int t = t0 + q;
        if (t < KK) {
          const int i = t / g.KW, j = t - (t / g.KW) * g.KW;
          const int ih = oh * g.SH - g.PH + i * g.DH;
          const int iw = ow * g.SW - g.PW + j * g.DW;
          unsigned xi = (unsigned)pad;
          if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
            xi = dw_index<T>(plane[ih * g.W + iw], offset);
          acc[q] += gv * stw[xi];
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) red[q][threadIdx.x] = acc[q];
    __syncthreads();
    if (threadIdx.x < 16 && t0 + (int)threadIdx.x < KK) {
      const int q = threadIdx.x;
      float a = 0.0f;
      for (int k = 0; k < DW_THREADS; ++k) a += red[q][k];
      ws[((long long)s * g.C + c) * KK + t0 + q] = a;
    }
    __syncthreads();
  }
}

static int dw_check(const atx_conv_geom& g, int dtype, int pad_index, const char* what) {
  int rc = check_geom(g);
  if (rc) return rc;
  ATX_REQUIRE(dtype >= 0 && dtype <= 3, "%s: bad dtype %d", what, dtype);
  ATX_REQUIRE(pad_index >= 0 && pad_index <= 255, "%s: bad pad_index", what);
  ATX_REQUIRE(g.KH * g.KW <= DW_MAX_TAPS, "%s: at most %d taps", what, DW_MAX_TAPS);
  ATX_REQUIRE(g.C <= 65535, "%s: C must be <= 65535", what);
  return ATX_OK;
}

template <typename T>
static void launch_dw_fwd(const T* img, const atx_conv_geom& g, int offset, int pad,
                          const uint8_t* wq, const uint16_t* l16, const float* lf32, int cls,
                          const DwEpilogue& ep, void* y, hipStream_t stream) {
  const int KK = g.KH * g.KW;
  const size_t smem = (size_t)KK * 256 * 4;
  const long long strips = (long long)g.N * g.OH * ((g.OW + 3) / 4);
  if (g.KW == 3 && g.DW == 1 && (g.SW == 1 || g.SW == 2) && strips < 0x7fffffffLL - 65536) {
    // about 2048 blocks in all, each a run of at least 256 strips (1024
    // outputs) of one channel, so the channel's table is staged once per run
    const long long per_c = std::max<long long>(1, cdiv(2048, g.C));
    const int chunk = (int)std::max<long long>(
        DW_THREADS, cdiv(cdiv(strips, per_c), DW_THREADS) * DW_THREADS);
    dim3 grid((unsigned)cdiv(strips, chunk), (unsigned)g.C);
    const bool vec = (g.OW & 3) == 0 && ((uintptr_t)y & 15) == 0;
    if constexpr (sizeof(T) == 1) {
      const long long bytes = (long long)g.N * g.C * g.H * g.W;
      if (g.KH == 3 && g.PW <= 4 && ((uintptr_t)img & 3) == 0 && (bytes & 3) == 0 &&
          bytes < 0x7fffffffLL - 64) {
        constexpr bool I8 = std::is_same<T, int8_t>::value;
#define ATX_DW_STRIP3(E, S, SWV)                                                           \
  hipLaunchKernelGGL((dwconv_fwd_strip3_kernel<E, S, I8, SWV, DW_STRIP_GROUP>), grid,   \
                     dim3(DW_THREADS), smem, stream, (const uint8_t*)img, g, pad, wq, l16, \
                     lf32, ep, y, chunk, vec)
#define ATX_DW_STRIP3S(SWV)                                                                \
        if (cls == ATX_LUT_F32) ATX_DW_STRIP3(float, false, SWV);                          \
        else if (cls == ATX_LUT_I16) ATX_DW_STRIP3(int, true, SWV);                        \
        else ATX_DW_STRIP3(int, false, SWV);
        if (g.SW == 1) {
          ATX_DW_STRIP3S(1)
        } else {
          ATX_DW_STRIP3S(2)
        }
#undef ATX_DW_STRIP3S
#undef ATX_DW_STRIP3
        return;
      }
    }
#define ATX_DW_STRIP(E, S, SWV)                                                              \
  hipLaunchKernelGGL((dwconv_fwd_strip_kernel<T, E, S, SWV>), grid, dim3(DW_THREADS), smem, \
                     stream, img, g, offset, pad, wq, l16, lf32, ep, y, chunk, vec)
#define ATX_DW_STRIPS(SWV)                                                                   \
    if (cls == ATX_LUT_F32) ATX_DW_STRIP(float, false, SWV);                                 \
    else if (cls == ATX_LUT_I16) ATX_DW_STRIP(int, true, SWV);                               \
    else ATX_DW_STRIP(int, false, SWV);
    if (g.SW == 1) {
      ATX_DW_STRIPS(1)
    } else {
      ATX_DW_STRIPS(2)
    }
#undef ATX_DW_STRIPS
#undef ATX_DW_STRIP
    return;
  }
  // about 2048 blocks in all, each a run of at least 1024 outputs of one
  // channel, so the channel's table is staged once per run
  const long long P = (long long)g.N * g.OH * g.OW;
  const long long per_c = std::max<long long>(1, cdiv(2048, g.C));
  const long long chunk = std::min<long long>(
      1LL << 30, std::max<long long>(1024, cdiv(cdiv(P, per_c), DW_THREADS) * DW_THREADS));
  dim3 grid((unsigned)cdiv(P, chunk), (unsigned)g.C);
  if (cls == ATX_LUT_F32)
    hipLaunchKernelGGL((dwconv_fwd_kernel<T, float, false>), grid, dim3(DW_THREADS), smem,
                       stream, img, g, offset, pad, wq, l16, lf32, ep, y, (int)chunk);
  else if (cls == ATX_LUT_I16)
    hipLaunchKernelGGL((dwconv_fwd_kernel<T, int, true>), grid, dim3(DW_THREADS), smem, stream,
                       img, g, offset, pad, wq, l16, lf32, ep, y, (int)chunk);
  else
    hipLaunchKernelGGL((dwconv_fwd_kernel<T, int, false>), grid, dim3(DW_THREADS), smem, stream,
                       img, g, offset, pad, wq, l16, lf32, ep, y, (int)chunk);
}

}  // namespace atx

using namespace atx;

extern "C" {

int atx_dwconv_fwd(const void* img, int dtype, atx_conv_geom g, int pad_index,
                   const uint8_t* wq, const uint16_t* lut16t, const float* lutf32t,
                   int lut_class, atx_gemm_epilogue ep, void* y, hipStream_t stream) {
  ATX_REQUIRE_EPILOGUE(ep, "atx_dwconv_fwd");
  int rc = dw_check(g, dtype, pad_index, "atx_dwconv_fwd");
  if (rc) return rc;
  ATX_REQUIRE(ep.out_kind >= ATX_OUT_F32 && ep.out_kind <= ATX_OUT_DEQUANT,
              "atx_dwconv_fwd: bad out_kind");
  ATX_REQUIRE(lut_class >= ATX_LUT_I16 && lut_class <= ATX_LUT_F32,
              "atx_dwconv_fwd: bad lut_class");
  ATX_REQUIRE(!(lut_class == ATX_LUT_F32 && ep.out_kind == ATX_OUT_I32),
              "atx_dwconv_fwd: int32 output needs an integer LUT");
  ATX_REQUIRE(ep.out_kind != ATX_OUT_DEQUANT || (ep.scale_x && ep.scale_w),
              "atx_dwconv_fwd: dequant epilogue needs scale_x and scale_w");
  if ((long long)g.N * g.C == 0) return ATX_OK;
  ATX_REQUIRE(img && wq && y && lut16t && lutf32t, "atx_dwconv_fwd: null pointer");
  const int offset = dtype == 3 ? 0 : 128;
  const DwEpilogue dep{ep.out_kind, ep.scale_x, ep.scale_w, ep.bias};
  if (dtype == 0)
    launch_dw_fwd<int8_t>((const int8_t*)img, g, offset, pad_index, wq, lut16t, lutf32t,
                          lut_class, dep, y, stream);
  else if (dtype == 1)
    launch_dw_fwd<uint8_t>((const uint8_t*)img, g, offset, pad_index, wq, lut16t, lutf32t,
                           lut_class, dep, y, stream);
  else
    launch_dw_fwd<float>((const float*)img, g, offset, pad_index, wq, lut16t, lutf32t,
                         lut_class, dep, y, stream);
  return check_launch("dwconv_fwd_kernel");
}

int atx_dwconv_bwd_data(const float* go, const uint8_t* wq, const float* tx, atx_conv_geom g,
                        const float* go_sx, const float* go_sw, const uint8_t* mask,
                        const float* scale, float* gx, hipStream_t stream) {
  int rc = dw_check(g, 0, 0, "atx_dwconv_bwd_data");
  if (rc) return rc;
  ATX_REQUIRE((go_sx == nullptr) == (go_sw == nullptr),
              "atx_dwconv_bwd_data: go_sx and go_sw come together");
  ATX_REQUIRE(!mask || scale, "atx_dwconv_bwd_data: mask needs scale");
  const long long total = (long long)g.N * g.C * g.H * g.W;
  if (total == 0) return ATX_OK;
  ATX_REQUIRE(go && wq && tx && gx, "atx_dwconv_bwd_data: null pointer");
  hipLaunchKernelGGL(dwconv_bwd_data_kernel, dim3(elem_grid(total, DW_THREADS)),
                     dim3(DW_THREADS), 0, stream, go, wq, tx, g, go_sx, go_sw, mask, scale, gx);
  return check_launch("dwconv_bwd_data_kernel");
}

long long atx_dwconv_bwd_weight_workspace_bytes(atx_conv_geom g) {
  const long long P = (long long)g.N * g.OH * g.OW;
  if (P <= 0 || g.C <= 0) return 0;
  return cdiv(P, DW_WSPLIT_ROWS) * g.C * g.KH * g.KW * 4;
}

int atx_dwconv_bwd_weight(const float* go, const void* img, int dtype, atx_conv_geom g,
                          int pad_index, const float* pad_dev, const float* tw,
                          const float* go_sx, const float* go_sw, const uint8_t* mask_w,
                          const float* scale_w, float* gw, float* workspace,
                          hipStream_t stream) {
  int rc = dw_check(g, dtype, pad_index, "atx_dwconv_bwd_weight");
  if (rc) return rc;
  ATX_REQUIRE((go_sx == nullptr) == (go_sw == nullptr),
              "atx_dwconv_bwd_weight: go_sx and go_sw come together");
  ATX_REQUIRE(!mask_w || scale_w, "atx_dwconv_bwd_weight: mask_w needs scale_w");
  const int KK = g.KH * g.KW;
  const long long numel = (long long)g.C * KK;
  if (numel == 0) return ATX_OK;
  ATX_REQUIRE(gw && tw, "atx_dwconv_bwd_weight: null pointer");
  const long long P = (long long)g.N * g.OH * g.OW;
  if (P == 0) return launch_split_sum(nullptr, 0, numel, KK, nullptr, nullptr, gw, stream);
  ATX_REQUIRE(go && img && workspace, "atx_dwconv_bwd_weight: null operand/workspace");
  const long long S = cdiv(P, DW_WSPLIT_ROWS);
  ATX_REQUIRE(S <= 65535, "atx_dwconv_bwd_weight: N*OH*OW too large");
  const int offset = dtype == 3 ? 0 : 128;
  dim3 grid((unsigned)g.C, (unsigned)S);
  if (dtype == 0)
    hipLaunchKernelGGL(dwconv_bwd_weight_kernel<int8_t>, grid, dim3(DW_THREADS), 0, stream,
                       go, (const int8_t*)img, g, offset, pad_index, pad_dev, tw, go_sx, go_sw,
                       workspace);
  else if (dtype == 1)
    hipLaunchKernelGGL(dwconv_bwd_weight_kernel<uint8_t>, grid, dim3(DW_THREADS), 0, stream,
                       go, (const uint8_t*)img, g, offset, pad_index, pad_dev, tw, go_sx, go_sw,
                       workspace);
  else
    hipLaunchKernelGGL(dwconv_bwd_weight_kernel<float>, grid, dim3(DW_THREADS), 0, stream,
                       go, (const float*)img, g, offset, pad_index, pad_dev, tw, go_sx, go_sw,
                       workspace);
  rc = check_launch("dwconv_bwd_weight_kernel");
  if (rc) return rc;
  return launch_split_sum(workspace, (int)S, numel, KK, mask_w, scale_w, gw, stream);
}

}  // extern "C"
