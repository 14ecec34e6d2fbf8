// Image -> LUT-index operands (implicit im2col), LUT maps and col2im (fold).
// All HBM-bound index arithmetic; k order is (c, kh, kw), l = oh*OW + ow.

#include "atx_internal.h"

#include <algorithm>

namespace atx {

constexpr int TB = 256;

// Index of one image element: int8 values index as v + 128, uint8 values as
// v, fp32 quantized values as clamp(rint(v), -128, 127) + 128 (the fp32
// convention of csrc/claude/bgemm_lre_backward_claude.cu:64-78).
template <typename T> __device__ __forceinline__ unsigned elem_index(T v, int offset);
template <> __device__ __forceinline__ unsigned elem_index<int8_t>(int8_t v, int) {
  return (unsigned)((int)v + 128);
}
template <> __device__ __forceinline__ unsigned elem_index<uint8_t>(uint8_t v, int) {
  return (unsigned)v;
}
template <> __device__ __forceinline__ unsigned elem_index<float>(float v, int offset) {
  return quant_index(v, offset);
}

// xt[slot][r] = row_offset(index of tap operand_tap(slot, r) at output
// position r); rows r >= N*L and taps k >= K hold 0.  A thread owns one quad
// of rows (four output positions, decomposed once) and walks the block's
// run of slots, writing the quad of each slot as one 8-byte store
// (consecutive threads: consecutive 8-byte pieces of a slot row).  The taps
// of the block's slots (channel, kh, kw) are decomposed once into an LDS
// table; slot s of quad q holds tap (s & ~3) | ((q + s) & 3).  The run is
// `slots` long (a multiple of 4, at most IM_SLOTS): shorter runs give small
// images (few row quads) more blocks.  PW4 (byte images of a 1x1, stride-1,
// unpadded conv with L % 4 == 0 and a 4-byte aligned image): a row quad is
// four consecutive bytes of each channel plane, read with one 4-byte load
// per tap (the int8 index v + 128 of byte b is b ^ 0x80).
constexpr int IM_SLOTS = 32;
template <typename T, bool PW4 = false>
__global__ void __launch_bounds__(TB)
im2col_rows_kernel(const T* __restrict__ img, atx_conv_geom g, int offset, int pad_index,
                   const float* __restrict__ pad_dev, uint16_t* __restrict__ xt, int Rpad,
                   int slots) {
  __shared__ int toff[IM_SLOTS];             // c*H*W + kh*DH*W + kw*DW
  __shared__ int tdh[IM_SLOTS], tdw[IM_SLOTS];
  const int KK = g.KH * g.KW;
  const int K = g.C * KK;
  const int HW = g.H * g.W;
  const int k0 = blockIdx.y * slots;
  if (threadIdx.x < slots) {
    const int k = min(k0 + (int)threadIdx.x, K - 1);
    const int c = k / KK, t = k - c * KK;
    const int kh = t / g.KW, kw = t - kh * g.KW;
    tdh[threadIdx.x] = kh * g.DH;
    tdw[threadIdx.x] = kw * g.DW;
    toff[threadIdx.x] = c * HW + kh * g.DH * g.W + kw * g.DW;
  }
  __syncthreads();
  const int q = blockIdx.x * TB + threadIdx.x;
  if (q >= (Rpad >> 2)) return;
  if (pad_dev) pad_index = (int)quant_index(pad_dev[0], 0);
  const int L = g.OH * g.OW;
  const int R = g.N * L;
  const int r0 = q << 2;
  // the quad's four output positions
  long long base[4];
  int ihb[4], iwb[4];
  unsigned valid = 0;
  {
    int n = min(r0, max(R - 1, 0)) / L;
    const int l = min(r0, max(R - 1, 0)) - n * L;
    int oh = l / g.OW, ow = l - oh * g.OW;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (r0 + e < R) valid |= 1u << e;
      ihb[e] = oh * g.SH - g.PH;
      iwb[e] = ow * g.SW - g.PW;
      base[e] = (long long)n * g.C * HW + (long long)ihb[e] * g.W + iwb[e];
      if (++ow == g.OW) { ow = 0; if (++oh == g.OH) { oh = 0; ++n; } }
    }
  }
  const int nslots = min(slots, operand_rows(K) - k0);   // a multiple of 4
  uint16_t* dst = xt + (long long)k0 * Rpad + r0;
  if constexpr (PW4) {
    const unsigned flip = offset == 128 ? 0x80808080u : 0u;
    for (int s4 = 0; s4 < nslots; s4 += 4) {
      unsigned w4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int kl = s4 | ((q + u) & 3);
        const bool b = k0 + kl < K && valid;   // L % 4 == 0: a quad is all rows or none
        w4[u] = b ? *(const unsigned*)(img + base[0] + toff[kl]) ^ flip : 0u;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool b = k0 + (s4 | ((q + u) & 3)) < K && valid;
        unsigned off[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) off[e] = b ? row_offset((w4[u] >> (8 * e)) & 255u) : 0u;
        *(uint2*)(dst + (long long)(s4 + u) * Rpad) =
            make_uint2(off[0] | (off[1] << 16), off[2] | (off[3] << 16));
      }
    }
    return;
  }
  for (int s4 = 0; s4 < nslots; s4 += 4) {
    // one quad of taps per iteration: its 16 loads are in flight together
    T raw[4][4];
    unsigned in = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int kl = s4 | ((q + u) & 3);        // this quad's tap of slot k0 + s4 + u
      const bool kv = k0 + kl < K;
      const int dh = tdh[kl], dw = tdw[kl], to = toff[kl];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ih = ihb[e] + dh, iw = iwb[e] + dw;
        // rows past R (padding) load nothing: their position may lie past
        // the last image
        const bool b = kv && ((valid >> e) & 1u) && (unsigned)ih < (unsigned)g.H &&
                       (unsigned)iw < (unsigned)g.W;
        raw[u][e] = img[b ? base[e] + to : 0];
        in |= (b ? 1u : 0u) << (4 * u + e);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool kv = k0 + (s4 | ((q + u) & 3)) < K;
      unsigned off[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const unsigned v = (in >> (4 * u + e)) & 1u ? elem_index<T>(raw[u][e], offset)
                                                    : (unsigned)pad_index;
        off[e] = kv && ((valid >> e) & 1u) ? row_offset(v) : 0u;
      }
      *(uint2*)(dst + (long long)(s4 + u) * Rpad) =
          make_uint2(off[0] | (off[1] << 16), off[2] | (off[3] << 16));
    }
  }
}

// The reference's im2col_u8 op: out[n][k][l] = index, padding -> 128.
template <typename T>
__global__ void im2col_u8_kernel(const T* __restrict__ img, atx_conv_geom g,
                                 uint8_t* __restrict__ out) {
  const int L = g.OH * g.OW;
  const int KK = g.KH * g.KW;
  const int K = g.C * KK;
  for (int k = blockIdx.y; k < K; k += gridDim.y) {
    const int c = k / KK;
    const int t = k - c * KK;
    const int kh = t / g.KW;
    const int kw = t - kh * g.KW;
    const int ih0 = kh * g.DH - g.PH;
    const int iw0 = kw * g.DW - g.PW;
    for (int n = blockIdx.z; n < g.N; n += gridDim.z) {
      uint8_t* o = out + ((long long)n * K + k) * L;
      for (int l = blockIdx.x * blockDim.x + threadIdx.x; l < L;
           l += gridDim.x * blockDim.x) {
        const int oh = l / g.OW;
        const int ow = l - oh * g.OW;
        const int ih = oh * g.SH + ih0;
        const int iw = ow * g.SW + iw0;
        unsigned v = 128u;
        if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
          v = elem_index<T>(img[(((long long)n * g.C + c) * g.H + ih) * g.W + iw], 128);
        o[l] = (uint8_t)v;
      }
    }
  }
}

template <typename T>
__global__ void lut_map_kernel(const T* __restrict__ in, long long n,
                               const float* __restrict__ lut, float* __restrict__ out) {
  __shared__ float sl[256];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) sl[i] = lut[i];
  __syncthreads();
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = sl[elem_index<T>(in[i], 128)];
}

template <typename T>
__global__ void lut_map_pad_kernel(const T* __restrict__ in, int N, int C, int H, int W,
                                   int PH, int PW, const float* __restrict__ lut,
                                   float* __restrict__ out) {
  __shared__ float sl[256];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) sl[i] = lut[i];
  __syncthreads();
  const int HP = H + 2 * PH, WP = W + 2 * PW;
  const long long n = (long long)N * C * HP * WP;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) {
    const int wp = (int)(i % WP);
    const long long t = i / WP;
    const int hp = (int)(t % HP);
    const long long nc = t / HP;
    const int h = hp - PH, w = wp - PW;
    float v = sl[128];
    if ((unsigned)h < (unsigned)H && (unsigned)w < (unsigned)W)
      v = sl[elem_index<T>(in[(nc * H + h) * W + w], 128)];
    out[i] = v;
  }
}

// col2im: img[n,c,h,w] = sum over taps (kh,kw) hitting (h,w) of
// col[n, (c,kh,kw), (oh,ow)], taps in ascending (kh, kw) order (F.fold).
// Optional per-position term: pos [N][L] (nullable) adds, as a second sum in
// the same tap order, sum over the hitting taps of pos[n, (oh,ow)] (the
// backward of a per-position term broadcast over a position's taps).
// Optional fused STE: img = mask ? img / s : 0 (s = max(scale[0], 1e-12)).
// One thread per image element; I = int when the image has fewer than 2^31
// elements (32-bit index arithmetic), long long otherwise.  The taps are
// loaded in batches of CT with no branches (a tap that does not hit the
// element loads element 0 and is skipped in the sum), so a thread has CT
// loads in flight; the sum keeps ascending (kh, kw) order (CT = 1 for a
// one-tap kernel).  ST = 1 when both strides are 1 (no divisions), 0 for
// the general case; both strides 2 take col2im_s2_kernel.
template <typename I, int ST, int CT>
__global__ void __launch_bounds__(TB)
col2im_kernel(const float* __restrict__ col, atx_conv_geom g, const float* __restrict__ pos,
              const uint8_t* __restrict__ mask, const float* __restrict__ scale,
              float* __restrict__ img) {
  const int L = g.OH * g.OW;
  const int KK = g.KH * g.KW;
  const I HW = (I)g.H * g.W;
  const I total = (I)g.N * g.C * HW;
  const float s = mask ? fmaxf(scale[0], 1e-12f) : 1.0f;
  for (I i = (I)blockIdx.x * TB + threadIdx.x; i < total; i += (I)gridDim.x * TB) {
    const I plane = i / HW;                   // n * C + c
    const int p = (int)(i - plane * HW);
    const int h = p / g.W, w = p - h * g.W;
    const float* cn = col + (long long)plane * KK * L;   // col[n][c*KK ..][L]
    const float* pn = pos ? pos + (long long)(plane / g.C) * L : nullptr;
    float a = 0.0f, b = 0.0f;
    int kh = 0, kw = 0;
    for (int t0 = 0; t0 < KK; t0 += CT) {
      float v[CT];
      int at[CT];
      unsigned ok = 0;
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        const int y = h + g.PH - kh * g.DH, x = w + g.PW - kw * g.DW;
        int oh, ow;
        bool hit;
        if constexpr (ST == 1) {
          oh = y; ow = x;
          hit = true;
        } else {
          oh = y >= 0 ? y / g.SH : 0; ow = x >= 0 ? x / g.SW : 0;
          hit = oh * g.SH == y && ow * g.SW == x;
        }
        hit = hit && t0 + j < KK && y >= 0 && x >= 0 && oh < g.OH && ow < g.OW;
        at[j] = hit ? oh * g.OW + ow : 0;
        v[j] = cn[hit ? (long long)(t0 + j) * L + at[j] : 0];
        ok |= (hit ? 1u : 0u) << j;
        if (++kw == g.KW) { kw = 0; ++kh; }
      }
#pragma unroll
      for (int j = 0; j < CT; ++j)
        if ((ok >> j) & 1u) a += v[j];
      if (pn) {
#pragma unroll
        for (int j = 0; j < CT; ++j)
          if ((ok >> j) & 1u) b += pn[at[j]];
      }
    }
    if (pn) a += b;
    if (mask) a = (mask[i] ? a : 0.0f) / s;
    img[i] = a;
  }
}

// col2im with at most 9 taps and stride 1, one thread per pixel position
// (n, h, w) and run of CC channels (blockIdx.y): the taps that reach the
// position, their col offsets and the position-term sum (the same for every
// channel, in the same ascending tap order) are worked out once and reused
// for each channel, whose tap loads, mask byte and store are then coalesced
// across the threads (consecutive w).  The same values as col2im_kernel.
// Taken when a position term is given: c5-shape 3 x 3 layers at batch 128
// take 225 / 124 / 55 / 27 us against 424 / 200 / 87 / 43 us for
// col2im_kernel, which re-reads the position term per channel; without one
// the two kernels are within 5% of each other and col2im_kernel stays.
constexpr int C2_CC = 16;
template <typename I>
__global__ void __launch_bounds__(TB)
col2im_cc_kernel(const float* __restrict__ col, atx_conv_geom g, const float* __restrict__ pos,
                 const uint8_t* __restrict__ mask, const float* __restrict__ scale,
                 float* __restrict__ img) {
  const int L = g.OH * g.OW;
  const int KK = g.KH * g.KW;
  const int HW = g.H * g.W;
  const I total = (I)g.N * HW;
  const float s = mask ? fmaxf(scale[0], 1e-12f) : 1.0f;
  const int c0 = blockIdx.y * C2_CC, nc = min(g.C - c0, C2_CC);
  for (I i = (I)blockIdx.x * TB + threadIdx.x; i < total; i += (I)gridDim.x * TB) {
    const I n = i / HW;
    const int p = (int)(i - n * HW);
    const int h = p / g.W, w = p - h * g.W;
    int at[9];
    unsigned ok = 0;
    int kh = 0, kw = 0;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const int oh = h + g.PH - kh * g.DH, ow = w + g.PW - kw * g.DW;
      const bool hit = j < KK && oh >= 0 && ow >= 0 && oh < g.OH && ow < g.OW;
      at[j] = hit ? j * L + oh * g.OW + ow : 0;
      ok |= (hit ? 1u : 0u) << j;
      if (++kw == g.KW) { kw = 0; ++kh; }
    }
    float b = 0.0f;
    if (pos) {
      const float* pn = pos + (long long)n * L;
      float u[9];
#pragma unroll
      for (int j = 0; j < 9; ++j) u[j] = pn[(ok >> j) & 1u ? at[j] - j * L : 0];
#pragma unroll
      for (int j = 0; j < 9; ++j)
        if ((ok >> j) & 1u) b += u[j];
    }
    for (int cc = 0; cc < nc; ++cc) {
      const I plane = n * g.C + c0 + cc;
      const float* cn = col + (long long)plane * KK * L;
      float v[9];
#pragma unroll
      for (int j = 0; j < 9; ++j) v[j] = cn[at[j]];
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < 9; ++j)
        if ((ok >> j) & 1u) a += v[j];
      if (pos) a += b;
      const I idx = plane * HW + p;
      if (mask) a = (mask[idx] ? a : 0.0f) / s;
      img[idx] = a;
    }
  }
}

// col2im with both strides 2, one thread per 2 x 2 block of pixels (rows
// 2a, 2a + 1, columns 2b, 2b + 1).  Pixel row h = 2a + e is reached by tap
// row kh when h + PH - kh * DH is even, i.e. for e = (PH - kh * DH) & 1
// whatever a: every tap feeds exactly one pixel of the block, and the lanes
// (consecutive b) read consecutive col elements for it.  Each pixel sums its
// taps in the same ascending (kh, kw) order as col2im_kernel: a tap that
// misses it adds +0, which leaves a sum started at +0 unchanged (such a sum
// is never -0).  A pixel that no tap reaches is +0 with or without its mask
// (0 / s), so its mask byte is not read.  VEC: W is even and img 8-byte
// aligned, so a block row is one 8-byte store.
template <typename I, int CT, bool VEC>
__global__ void __launch_bounds__(TB)
col2im_s2_kernel(const float* __restrict__ col, atx_conv_geom g, const float* __restrict__ pos,
                 const uint8_t* __restrict__ mask, const float* __restrict__ scale,
                 float* __restrict__ img) {
  const int L = g.OH * g.OW;
  const int KK = g.KH * g.KW;
  const int H2 = (g.H + 1) >> 1, W2 = (g.W + 1) >> 1;
  const I B2 = (I)H2 * W2;
  const I HW = (I)g.H * g.W;
  const I total = (I)g.N * g.C * B2;
  const float s = mask ? fmaxf(scale[0], 1e-12f) : 1.0f;
  for (I i = (I)blockIdx.x * TB + threadIdx.x; i < total; i += (I)gridDim.x * TB) {
    const I plane = i / B2;                   // n * C + c
    const int q = (int)(i - plane * B2);
    const int a = q / W2, b = q - a * W2;
    const float* cn = col + (long long)plane * KK * L;
    const float* pn = pos ? pos + (long long)(plane / g.C) * L : nullptr;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, pb[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    unsigned any = 0;                         // pixels of the block some tap reaches
    int kh = 0, kw = 0;
    for (int t0 = 0; t0 < KK; t0 += CT) {
      float v[CT], u[CT];
      int e[CT];
      bool ok[CT];
#pragma unroll
      for (int j = 0; j < CT; ++j) {
        const int yb = g.PH - kh * g.DH, xb = g.PW - kw * g.DW;
        const int eh = yb & 1, ew = xb & 1;   // the block row and column the tap reaches
        const int y = 2 * a + eh + yb, x = 2 * b + ew + xb;   // both even
        const int oh = y >> 1, ow = x >> 1;
        ok[j] = t0 + j < KK && y >= 0 && x >= 0 && oh < g.OH && ow < g.OW &&
                2 * a + eh < g.H && 2 * b + ew < g.W;
        const int at = ok[j] ? oh * g.OW + ow : 0;
        v[j] = cn[ok[j] ? (long long)(t0 + j) * L + at : 0];
        u[j] = pn ? pn[at] : 0.0f;
        e[j] = 2 * eh + ew;
        if (++kw == g.KW) { kw = 0; ++kh; }
      }
#pragma unroll
      for (int j = 0; j < CT; ++j) {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += ok[j] && e[j] == c ? v[j] : 0.0f;
        any |= (ok[j] ? 1u : 0u) << e[j];
      }
      if (pn) {
#pragma unroll
        for (int j = 0; j < CT; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) pb[c] += ok[j] && e[j] == c ? u[j] : 0.0f;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (pn) acc[c] += pb[c];
      if (mask && ((any >> c) & 1u)) {
        const I idx = plane * HW + (I)(2 * a + (c >> 1)) * g.W + 2 * b + (c & 1);
        acc[c] = (mask[idx] ? acc[c] : 0.0f) / s;
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int h = 2 * a + r;
      if (h >= g.H) break;
      const I idx = plane * HW + (I)h * g.W + 2 * b;
      if constexpr (VEC) {
        *(float2*)(img + idx) = make_float2(acc[2 * r], acc[2 * r + 1]);
      } else {
        img[idx] = acc[2 * r];
        if (2 * b + 1 < g.W) img[idx + 1] = acc[2 * r + 1];
      }
    }
  }
}

// Sum over the K taps of each output position (out-of-image taps count as
// pad_dev[0]): the column sums of the unfolded image, used by the uint8
// zero-point correction (nn/Conv2d_uint8.py:311).
// Column sums of the unfolded image in two phases (every sum is of
// quantized integers below 2^24, so exact in any order):
//   partial[n][chunk][h*W + w] = sum over the chunk's 64 channels of img,
//   out[n,l] = sum over the KH*KW taps of output position l of the chunk sums
//              at the tap's pixel, or C * pad for a tap outside the image.
constexpr int TS_CHUNK = 64;

template <typename T>
__global__ void tap_chan_sum_kernel(const T* __restrict__ img, int C, int HW, int chunks,
                                    long long total, float* __restrict__ partial) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
    const int p = (int)(i % HW);
    const long long t = i / HW;
    const int ch = (int)(t % chunks);
    const int n = (int)(t / chunks);
    const int nc = min(C - ch * TS_CHUNK, TS_CHUNK);
    const T* src = img + ((long long)n * C + ch * TS_CHUNK) * HW + p;
    float a = 0.0f;
    int c = 0;
    for (; c + 16 <= nc; c += 16) {           // 16 channels' loads in flight, added in order
      T v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = src[(long long)(c + j) * HW];
#pragma unroll
      for (int j = 0; j < 16; ++j) a += (float)v[j];
    }
    for (; c < nc; ++c) a += (float)src[(long long)c * HW];
    partial[i] = a;
  }
}

// The same chunk sums for a byte image whose planes are 4-byte aligned
// (H * W % 4 == 0): a thread owns four consecutive pixels and reads them
// with one 4-byte load per channel, 16 channels' loads in flight.  The
// bytes are summed two to a register in 16-bit fields (even bytes, odd
// bytes; at most 64 * 255 = 16320 per field, so no carry crosses a field):
// the integer sums, converted once, are the values tap_chan_sum_kernel's
// fp32 sums of integers below 2^24 give.
__global__ void __launch_bounds__(256)
tap_chan_sum_u8x4_kernel(const uint8_t* __restrict__ img, int C, int HW, int chunks,
                         long long total4, float* __restrict__ partial) {
  constexpr int U = 16;
  const int HW4 = HW >> 2;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total4; i += stride) {
    const int p4 = (int)(i % HW4);
    const long long t = i / HW4;
    const int ch = (int)(t % chunks);
    const long long n = t / chunks;
    const int c0 = ch * TS_CHUNK, nc = min(C - c0, TS_CHUNK);
    const unsigned* src = (const unsigned*)(img + (n * C + c0) * HW) + p4;
    unsigned ev = 0, od = 0;                  // bytes 0 and 2 / 1 and 3, 16 bits each
    int c = 0;
    for (; c + U <= nc; c += U) {
      unsigned v[U];
#pragma unroll
      for (int j = 0; j < U; ++j) v[j] = src[(long long)(c + j) * HW4];
#pragma unroll
      for (int j = 0; j < U; ++j) {
        ev += v[j] & 0x00ff00ffu;
        od += (v[j] >> 8) & 0x00ff00ffu;
      }
    }
    for (; c < nc; ++c) {
      const unsigned v = src[(long long)c * HW4];
      ev += v & 0x00ff00ffu;
      od += (v >> 8) & 0x00ff00ffu;
    }
    *(float4*)(partial + 4 * i) = make_float4((float)(ev & 0xffffu), (float)(od & 0xffffu),
                                              (float)(ev >> 16), (float)(od >> 16));
  }
}

__global__ void tap_window_sum_kernel(const float* __restrict__ partial, atx_conv_geom g,
                                      int chunks, const float* __restrict__ pad_dev,
                                      float* __restrict__ out) {
  const int L = g.OH * g.OW, HW = g.H * g.W;
  const long long total = (long long)g.N * L;
  const float padc = (pad_dev ? pad_dev[0] : 0.0f) * (float)g.C;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
    const int n = (int)(i / L), l = (int)(i - (i / L) * L);
    const int oh = l / g.OW, ow = l - (l / g.OW) * g.OW;
    const float* pn = partial + (long long)n * chunks * HW;
    float a = 0.0f;
    for (int kh = 0; kh < g.KH; ++kh) {
      const int ih = oh * g.SH + kh * g.DH - g.PH;
      for (int kw = 0; kw < g.KW; ++kw) {
        const int iw = ow * g.SW + kw * g.DW - g.PW;
        if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W) {
          for (int ch = 0; ch < chunks; ++ch) a += pn[(long long)ch * HW + ih * g.W + iw];
        } else {
          a += padc;
        }
      }
    }
    out[i] = a;
  }
}

// The uint8 layer's zero-point position term in backward:
// pos[n,l] = sum_o coef[o] * go[n,o,l], coef[o] = -((sx * sw[o]) * zw[o])
// (the fp32 products of -(scale_x * scale_w) * zero_w).  A block owns P
// positions of one image (blockIdx.y) and G channel groups (P * G = 256):
// thread (p, gi) sums the channels gi, gi + G, ... of position p (loads of
// P consecutive positions per channel are coalesced), then the G partials
// are combined in a fixed order through LDS, so results are identical run to
// run.  P = 64 for L >= 64, else 16 (small images: more channel groups).
template <int P>
__global__ void __launch_bounds__(256)
channel_dot_kernel(const float* __restrict__ go, int O, int L, const float* __restrict__ sx,
                   const float* __restrict__ sw, const float* __restrict__ zw,
                   float* __restrict__ pos) {
  constexpr int G = 256 / P;
  __shared__ float part[G][P];
  const int p = threadIdx.x % P, gi = threadIdx.x / P;
  const int l = blockIdx.x * P + p;
  const long long n = blockIdx.y;
  const float s = sx[0];
  float acc = 0.0f;
  if (l < L) {
    const float* src = go + n * O * L + l;
#pragma unroll 4
    for (int o = gi; o < O; o += G) {
      const float c = -((s * sw[o]) * zw[o]);
      acc += c * src[(long long)o * L];
    }
  }
  part[gi][p] = acc;
  __syncthreads();
  if (gi == 0 && l < L) {
    float t = part[0][p];
#pragma unroll
    for (int j = 1; j < G; ++j) t += part[j][p];
    pos[n * L + l] = t;
  }
}

// v + the value of the lane that DPP control CTRL picks (0 in the rows that
// ROW_MASK leaves out).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(
                 __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum of v over a group of P lanes in a fixed order: pairs (quad_perm
// [1,0,3,2]), quads ([2,3,0,1]), half rows (row_half_mirror), rows of 16
// (row_mirror) -- every lane of a row then holds the row's sum -- and for
// P = 64 rows 0+1 and 2+3 (row_bcast15 into rows 1 and 3), then all four
// (row_bcast31 into row 3): the wave's sum is in lane 63.
template <int P>
__device__ __forceinline__ float group_sum(float v) {
  v = dpp_add<0xB1, 0xf>(v);
  v = dpp_add<0x4E, 0xf>(v);
  v = dpp_add<0x141, 0xf>(v);
  v = dpp_add<0x140, 0xf>(v);
  if constexpr (P == 64) {
    v = dpp_add<0x142, 0xa>(v);
    v = dpp_add<0x143, 0xc>(v);
  }
  return v;
}

// Both zero-point reductions of go in one pass: pos[n,l] as
// channel_dot_kernel (the same products and order, so the same bits) when
// POS, and per-channel sums of go when SUM.  Persistent blocks walk the
// (image, P-position chunk) pairs blockIdx.x, + gridDim.x, ...; a chunk's
// value of channel o is summed over its P positions by group_sum and added
// by one lane to the block's total chs[o] in LDS (channel o belongs to group
// o % G only: each total has one writer lane, whose LDS adds take effect in
// program order, so the sums are the same run to run).  At the end each block
// writes its totals to part[blockIdx.x][O]; chan_total_kernel sums them.
// Loads: U channels per group in flight per thread.
template <int P, bool POS, bool SUM>
__global__ void __launch_bounds__(256)
zero_point_terms_kernel(const float* __restrict__ go, int N, int O, int L,
                        const float* __restrict__ sx, const float* __restrict__ sw,
                        const float* __restrict__ zw, float* __restrict__ pos,
                        float* __restrict__ part) {
  constexpr int G = 256 / P;
  constexpr int U = 8;
  constexpr int LAST = P == 64 ? 63 : 0;        // the lane that holds a group's sum
  __shared__ float pp[G][P];
  extern __shared__ float chs[];                // [O]
  const int p = threadIdx.x % P, gi = threadIdx.x / P;
  const int nlb = (L + P - 1) / P;
  const long long total = (long long)N * nlb;
  const float s = POS ? sx[0] : 0.0f;
  if constexpr (SUM)
    for (int o = threadIdx.x; o < O; o += 256) chs[o] = 0.0f;
  __syncthreads();
  for (long long c = blockIdx.x; c < total; c += gridDim.x) {
    const long long n = c / nlb;
    const int l = (int)(c - n * nlb) * P + p;
    const bool in = l < L;
    const float* src = go + n * O * L + (in ? l : 0);
    float acc = 0.0f;
    for (int o0 = gi; o0 < O; o0 += G * U) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int o = o0 + G * u;
        v[u] = in && o < O ? src[(long long)o * L] : 0.0f;
      }
      if constexpr (POS) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int o = o0 + G * u;
          if (o < O) acc += -((s * sw[o]) * zw[o]) * v[u];
        }
      }
      if constexpr (SUM) {
        float t[U];
#pragma unroll
        for (int u = 0; u < U; ++u) t[u] = group_sum<P>(v[u]);
        if (p == LAST) {      // LDS adds without a return value: nothing waits on them
#pragma unroll
          for (int u = 0; u < U; ++u)
            if (o0 + G * u < O) atomicAdd(&chs[o0 + G * u], t[u]);
        }
      }
    }
    if constexpr (POS) {
      pp[gi][p] = acc;
      __syncthreads();
      if (gi == 0 && in) {
        float t = pp[0][p];
#pragma unroll
        for (int j = 1; j < G; ++j) t += pp[j][p];
        pos[n * L + l] = t;
      }
      __syncthreads();                          // pp is rewritten by the next chunk
    }
  }
  if constexpr (SUM) {
    __syncthreads();
    for (int o = threadIdx.x; o < O; o += 256) part[(long long)blockIdx.x * O + o] = chs[o];
  }
}

__global__ void zp_zero_kernel(float* __restrict__ out, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = 0.0f;
}

// gsum[o] = sum over b < nb of part[b][o]: 16 slices (b = s, s + 16, ...)
// per channel, combined in slice order (deterministic).
__global__ void __launch_bounds__(256)
chan_total_kernel(const float* __restrict__ part, int nb, int O, float* __restrict__ gsum) {
  __shared__ float sl[16][16];
  const int c = threadIdx.x % 16, sidx = threadIdx.x / 16;
  const int o = blockIdx.x * 16 + c;
  float a = 0.0f;
  if (o < O) {
#pragma unroll 8
    for (int b = sidx; b < nb; b += 16) a += part[(long long)b * O + o];
  }
  sl[sidx][c] = a;
  __syncthreads();
  if (sidx == 0 && o < O) {
    float t = sl[0][c];
#pragma unroll
    for (int j = 1; j < 16; ++j) t += sl[j][c];
    gsum[o] = t;
  }
}

// Backward of tap_sum: img_grad[n,c,h,w] = sum of go[n,l] over the taps
// (kh, kw) that read (h, w) (independent of c).
__global__ void tap_sum_bwd_kernel(const float* __restrict__ go, atx_conv_geom g,
                                   float* __restrict__ img) {
  const int L = g.OH * g.OW;
  const long long total = (long long)g.N * g.C * g.H * g.W;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
    const int w = (int)(i % g.W);
    long long t = i / g.W;
    const int h = (int)(t % g.H);
    const int n = (int)(t / g.H / g.C);
    const float* gn = go + (long long)n * L;
    float a = 0.0f;
    for (int kh = 0; kh < g.KH; ++kh) {
      const int y = h + g.PH - kh * g.DH;
      if (y < 0 || y % g.SH) continue;
      const int oh = y / g.SH;
      if (oh >= g.OH) continue;
      for (int kw = 0; kw < g.KW; ++kw) {
        const int x = w + g.PW - kw * g.DW;
        if (x < 0 || x % g.SW) continue;
        const int ow = x / g.SW;
        if (ow >= g.OW) continue;
        a += gn[oh * g.OW + ow];
      }
    }
    img[i] = a;
  }
}

int check_geom(const atx_conv_geom& g) {
  ATX_REQUIRE(g.N >= 0 && g.C >= 0 && g.H >= 0 && g.W >= 0, "conv geometry: negative size");
  ATX_REQUIRE(g.KH > 0 && g.KW > 0 && g.SH > 0 && g.SW > 0 && g.DH > 0 && g.DW > 0 &&
                  g.PH >= 0 && g.PW >= 0,
              "conv geometry: kernel/stride/dilation must be positive, padding >= 0");
  ATX_REQUIRE(g.OH == (g.H + 2 * g.PH - g.DH * (g.KH - 1) - 1) / g.SH + 1 &&
                  g.OW == (g.W + 2 * g.PW - g.DW * (g.KW - 1) - 1) / g.SW + 1,
              "conv geometry: OH/OW do not match the input geometry");
  ATX_REQUIRE(g.OH > 0 && g.OW > 0, "conv geometry: empty output");
  return ATX_OK;
}

}  // namespace atx

using namespace atx;

extern "C" {

int atx_im2col_rows(const void* img, int dtype, atx_conv_geom g, int pad_index,
                    const float* pad_dev, uint16_t* xt, int Rpad, hipStream_t stream) {
  int rc = check_geom(g);
  if (rc) return rc;
  ATX_REQUIRE(dtype >= 0 && dtype <= 3, "atx_im2col_rows: bad dtype %d", dtype);
  // dtype 2: fp32 signed quantized values (index v+128); 3: fp32 unsigned
  // quantized values (index v).
  const int offset = dtype == 3 ? 0 : 128;
  if (dtype == 3) dtype = 2;
  ATX_REQUIRE(pad_index >= 0 && pad_index <= 255, "atx_im2col_rows: bad pad_index");
  const long long R = (long long)g.N * g.OH * g.OW;
  ATX_REQUIRE(Rpad >= R && Rpad % ATX_ROW_TILE == 0, "atx_im2col_rows: bad Rpad %d", Rpad);
  const int K = g.C * g.KH * g.KW;
  if ((long long)K * Rpad == 0) return ATX_OK;
  ATX_REQUIRE(xt && (R == 0 || img), "atx_im2col_rows: null pointer");
  static_assert(IM_SLOTS % 4 == 0, "slot runs are whole quads of taps");
  // the longest slot run that still gives the chip 2048 blocks (8 per CU)
  const long long xblocks = cdiv(Rpad / 4, TB);
  int slots = IM_SLOTS;
  while (slots > 4 && xblocks * cdiv(operand_rows(K), slots) < 2048) slots >>= 1;
  ATX_REQUIRE(cdiv(operand_rows(K), slots) <= 65535, "atx_im2col_rows: K too large");
  dim3 grid((unsigned)xblocks, (unsigned)cdiv(operand_rows(K), slots));
  const bool pw4 = g.KH == 1 && g.KW == 1 && g.SH == 1 && g.SW == 1 && g.PH == 0 && g.PW == 0 &&
                   (g.H * g.W) % 4 == 0 && ((uintptr_t)img & 3) == 0;
  if (pw4 && dtype == 0)
    hipLaunchKernelGGL((im2col_rows_kernel<int8_t, true>), grid, dim3(TB), 0, stream,
                       (const int8_t*)img, g, 128, pad_index, pad_dev, xt, Rpad, slots);
  else if (pw4 && dtype == 1)
    hipLaunchKernelGGL((im2col_rows_kernel<uint8_t, true>), grid, dim3(TB), 0, stream,
                       (const uint8_t*)img, g, 0, pad_index, pad_dev, xt, Rpad, slots);
  else if (dtype == 0)
    hipLaunchKernelGGL(im2col_rows_kernel<int8_t>, grid, dim3(TB), 0, stream,
                       (const int8_t*)img, g, 128, pad_index, pad_dev, xt, Rpad, slots);
  else if (dtype == 1)
    hipLaunchKernelGGL(im2col_rows_kernel<uint8_t>, grid, dim3(TB), 0, stream,
                       (const uint8_t*)img, g, 0, pad_index, pad_dev, xt, Rpad, slots);
  else
    hipLaunchKernelGGL(im2col_rows_kernel<float>, grid, dim3(TB), 0, stream,
                       (const float*)img, g, offset, pad_index, pad_dev, xt, Rpad, slots);
  return check_launch("im2col_rows_kernel");
}

int atx_im2col_u8(const void* img, int dtype, atx_conv_geom g, uint8_t* out,
                  hipStream_t stream) {
  int rc = check_geom(g);
  if (rc) return rc;
  ATX_REQUIRE(dtype >= 0 && dtype <= 2, "atx_im2col_u8: bad dtype %d", dtype);
  const int K = g.C * g.KH * g.KW;
  const int L = g.OH * g.OW;
  if ((long long)g.N * K * L == 0) return ATX_OK;
  ATX_REQUIRE(img && out, "atx_im2col_u8: null pointer");
  dim3 grid((unsigned)std::min<long long>(cdiv(L, TB), 64), (unsigned)std::min(K, 65535),
            (unsigned)std::min(g.N, 64));
  if (dtype == 0)
    hipLaunchKernelGGL(im2col_u8_kernel<int8_t>, grid, dim3(TB), 0, stream,
                       (const int8_t*)img, g, out);
  else if (dtype == 1)
    hipLaunchKernelGGL(im2col_u8_kernel<uint8_t>, grid, dim3(TB), 0, stream,
                       (const uint8_t*)img, g, out);
  else
    hipLaunchKernelGGL(im2col_u8_kernel<float>, grid, dim3(TB), 0, stream,
                       (const float*)img, g, out);
  return check_launch("im2col_u8_kernel");
}

int atx_lut_map(const void* in, int dtype, long long n, const float* lut256, float* out,
                hipStream_t stream) {
  ATX_REQUIRE(n >= 0 && dtype >= 0 && dtype <= 2, "atx_lut_map: bad arguments");
  if (n == 0) return ATX_OK;
  ATX_REQUIRE(in && lut256 && out, "atx_lut_map: null pointer");
  const int grid = elem_grid(n, TB);
  if (dtype == 0)
    hipLaunchKernelGGL(lut_map_kernel<int8_t>, dim3(grid), dim3(TB), 0, stream,
                       (const int8_t*)in, n, lut256, out);
  else if (dtype == 1)
    hipLaunchKernelGGL(lut_map_kernel<uint8_t>, dim3(grid), dim3(TB), 0, stream,
                       (const uint8_t*)in, n, lut256, out);
  else
    hipLaunchKernelGGL(lut_map_kernel<float>, dim3(grid), dim3(TB), 0, stream,
                       (const float*)in, n, lut256, out);
  return check_launch("lut_map_kernel");
}

int atx_lut_map_pad(const void* in, int dtype, int N, int C, int H, int W, int PH, int PW,
                    const float* lut256, float* out, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && C >= 0 && H >= 0 && W >= 0 && PH >= 0 && PW >= 0 && dtype >= 0 &&
                  dtype <= 2,
              "atx_lut_map_pad: bad arguments");
  const long long n = (long long)N * C * (H + 2 * PH) * (W + 2 * PW);
  if (n == 0) return ATX_OK;
  ATX_REQUIRE(lut256 && out && ((long long)N * C * H * W == 0 || in), "atx_lut_map_pad: null");
  const int grid = elem_grid(n, TB);
  if (dtype == 0)
    hipLaunchKernelGGL(lut_map_pad_kernel<int8_t>, dim3(grid), dim3(TB), 0, stream,
                       (const int8_t*)in, N, C, H, W, PH, PW, lut256, out);
  else if (dtype == 1)
    hipLaunchKernelGGL(lut_map_pad_kernel<uint8_t>, dim3(grid), dim3(TB), 0, stream,
                       (const uint8_t*)in, N, C, H, W, PH, PW, lut256, out);
  else
    hipLaunchKernelGGL(lut_map_pad_kernel<float>, dim3(grid), dim3(TB), 0, stream,
                       (const float*)in, N, C, H, W, PH, PW, lut256, out);
  return check_launch("lut_map_pad_kernel");
}

long long atx_tap_sum_workspace_bytes(atx_conv_geom g) {
  if (g.N <= 0 || g.C <= 0 || g.H <= 0 || g.W <= 0) return 0;
  return (long long)g.N * cdiv(g.C, TS_CHUNK) * g.H * g.W * 4;
}

int atx_tap_sum(const void* img, int dtype, atx_conv_geom g, const float* pad_dev, float* out,
                float* workspace, hipStream_t stream) {
  int rc = check_geom(g);
  if (rc) return rc;
  ATX_REQUIRE(dtype == 1 || dtype == 2, "atx_tap_sum: dtype must be 1 (uint8) or 2 (fp32)");
  const long long total = (long long)g.N * g.OH * g.OW;
  if (total == 0) return ATX_OK;
  ATX_REQUIRE(out, "atx_tap_sum: null output");
  const int chunks = (int)cdiv(g.C, TS_CHUNK);
  const long long ptotal = (long long)g.N * chunks * g.H * g.W;
  if (ptotal > 0) {
    ATX_REQUIRE(img && workspace, "atx_tap_sum: null image / workspace");
    const int HW = g.H * g.W;
    if (dtype == 1 && HW % 4 == 0 && ((uintptr_t)img & 3) == 0 && ((uintptr_t)workspace & 15) == 0)
      hipLaunchKernelGGL(tap_chan_sum_u8x4_kernel, dim3(elem_grid(ptotal / 4, TB)), dim3(TB), 0,
                         stream, (const uint8_t*)img, g.C, HW, chunks, ptotal / 4, workspace);
    else if (dtype == 1)
      hipLaunchKernelGGL(tap_chan_sum_kernel<uint8_t>, dim3(elem_grid(ptotal, TB)), dim3(TB), 0,
                         stream, (const uint8_t*)img, g.C, HW, chunks, ptotal, workspace);
    else
      hipLaunchKernelGGL(tap_chan_sum_kernel<float>, dim3(elem_grid(ptotal, TB)), dim3(TB), 0,
                         stream, (const float*)img, g.C, g.H * g.W, chunks, ptotal, workspace);
    rc = check_launch("tap_chan_sum_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(tap_window_sum_kernel, dim3(elem_grid(total, TB)), dim3(TB), 0, stream,
                     workspace, g, g.C > 0 ? chunks : 0, pad_dev, out);
  return check_launch("tap_window_sum_kernel");
}

int atx_tap_sum_bwd(const float* go, atx_conv_geom g, float* img, hipStream_t stream) {
  int rc = check_geom(g);
  if (rc) return rc;
  const long long total = (long long)g.N * g.C * g.H * g.W;
  if (total == 0) return ATX_OK;
  ATX_REQUIRE(go && img, "atx_tap_sum_bwd: null pointer");
  hipLaunchKernelGGL(tap_sum_bwd_kernel, dim3(elem_grid(total, TB)), dim3(TB), 0, stream, go, g,
                     img);
  return check_launch("tap_sum_bwd_kernel");
}

int atx_zero_point_pos(const float* go, int N, int O, int L, const float* scale_x,
                       const float* scale_w, const float* zero_w, float* pos,
                       hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && O >= 0 && L >= 0, "atx_zero_point_pos: negative size");
  if ((long long)N * L == 0) return ATX_OK;
  ATX_REQUIRE(pos && scale_x && (O == 0 || (go && scale_w && zero_w)),
              "atx_zero_point_pos: null pointer");
  ATX_REQUIRE(N <= 65535, "atx_zero_point_pos: N must be at most 65535");
  if (L >= 64)
    hipLaunchKernelGGL(channel_dot_kernel<64>, dim3((unsigned)cdiv(L, 64), (unsigned)N),
                       dim3(256), 0, stream, go, O, L, scale_x, scale_w, zero_w, pos);
  else
    hipLaunchKernelGGL(channel_dot_kernel<16>, dim3((unsigned)cdiv(L, 16), (unsigned)N),
                       dim3(256), 0, stream, go, O, L, scale_x, scale_w, zero_w, pos);
  return check_launch("channel_dot_kernel");
}

// Blocks of zero_point_terms_kernel: enough resident waves to stream go,
// few enough partial rows for chan_total_kernel.
constexpr int ZP_BLOCKS = 2048;
constexpr int ZP_MAX_O = 8192;          // the per-block channel totals in LDS (32 KiB)

static long long zp_blocks(int N, int L) {
  const int P = L >= 64 ? 64 : 16;
  return std::max<long long>(1, std::min<long long>(ZP_BLOCKS, (long long)N * cdiv(L, P)));
}

long long atx_zero_point_terms_workspace_bytes(int N, int O, int L) {
  if (N <= 0 || O <= 0 || L <= 0) return 0;
  return zp_blocks(N, L) * O * (long long)sizeof(float);
}

int atx_zero_point_terms(const float* go, int N, int O, int L, const float* scale_x,
                         const float* scale_w, const float* zero_w, float* pos, float* gsum,
                         float* workspace, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && O >= 0 && L >= 0, "atx_zero_point_terms: negative size");
  ATX_REQUIRE(O <= ZP_MAX_O || !gsum, "atx_zero_point_terms: channel sums support at most %d channels",
              ZP_MAX_O);
  if (!gsum) return atx_zero_point_pos(go, N, O, L, scale_x, scale_w, zero_w, pos, stream);
  if (O == 0) return ATX_OK;
  const long long NL = (long long)N * L;
  if (NL == 0) {                          // empty sums; no positions to write
    hipLaunchKernelGGL(zp_zero_kernel, dim3(1), dim3(256), 0, stream, gsum, O);
    return check_launch("zp_zero_kernel");
  }
  ATX_REQUIRE(go && workspace && (!pos || (scale_x && scale_w && zero_w)),
              "atx_zero_point_terms: null pointer");
  const int nb = (int)zp_blocks(N, L);
  const size_t lds = (size_t)O * sizeof(float);
#define ATX_ZPT(P, POS)                                                                        \
  hipLaunchKernelGGL((zero_point_terms_kernel<P, POS, true>), dim3(nb), dim3(256), lds, stream, \
                     go, N, O, L, scale_x, scale_w, zero_w, pos, workspace)
  if (L >= 64) { if (pos) ATX_ZPT(64, true); else ATX_ZPT(64, false); }
  else { if (pos) ATX_ZPT(16, true); else ATX_ZPT(16, false); }
#undef ATX_ZPT
  int rc = check_launch("zero_point_terms_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(chan_total_kernel, dim3((unsigned)cdiv(O, 16)), dim3(256), 0, stream,
                     workspace, nb, O, gsum);
  return check_launch("chan_total_kernel");
}

int atx_col2im(const float* col, atx_conv_geom g, const uint8_t* mask, const float* scale,
               float* img, hipStream_t stream) {
  return atx_col2im_pos(col, g, nullptr, mask, scale, img, stream);
}

int atx_col2im_pos(const float* col, atx_conv_geom g, const float* pos, const uint8_t* mask,
                   const float* scale, float* img, hipStream_t stream) {
  int rc = check_geom(g);
  if (rc) return rc;
  const long long total = (long long)g.N * g.C * g.H * g.W;
  if (total == 0) return ATX_OK;
  ATX_REQUIRE(col && img && (!mask || scale), "atx_col2im: null pointer");
  const dim3 grid(elem_grid(total, TB));
  const bool small = total < 0x7fffffffLL - (long long)grid.x * TB;
  const int st = g.SH == g.SW && (g.SH == 1 || g.SH == 2) ? g.SH : 0;
  const bool one = g.KH * g.KW == 1;
#define ATX_COL2IM(I, S, C)                                                              \
  hipLaunchKernelGGL((col2im_kernel<I, S, C>), grid, dim3(TB), 0, stream, col, g, pos,    \
                     mask, scale, img)
  if (!small) ATX_COL2IM(long long, 0, 9);
  else if (st == 1 && !one && g.KH * g.KW <= 9 && pos && cdiv(g.C, C2_CC) <= 65535) {
    const dim3 grid_cc(elem_grid((long long)g.N * g.H * g.W, TB), (unsigned)cdiv(g.C, C2_CC));
    hipLaunchKernelGGL(col2im_cc_kernel<int>, grid_cc, dim3(TB), 0, stream, col, g, pos, mask,
                       scale, img);
  }
  else if (st == 1) { if (one) ATX_COL2IM(int, 1, 1); else ATX_COL2IM(int, 1, 9); }
  else if (st == 2) {
    const dim3 grid2(elem_grid((long long)g.N * g.C * ((g.H + 1) / 2) * ((g.W + 1) / 2), TB));
    const bool vec = g.W % 2 == 0 && ((uintptr_t)img & 7) == 0;
#define ATX_COL2IM_S2(C, V)                                                                 \
  hipLaunchKernelGGL((col2im_s2_kernel<int, C, V>), grid2, dim3(TB), 0, stream, col, g, pos, \
                     mask, scale, img)
    if (one) { if (vec) ATX_COL2IM_S2(1, true); else ATX_COL2IM_S2(1, false); }
    else { if (vec) ATX_COL2IM_S2(9, true); else ATX_COL2IM_S2(9, false); }
#undef ATX_COL2IM_S2
  }
  else { if (one) ATX_COL2IM(int, 0, 1); else ATX_COL2IM(int, 0, 9); }
#undef ATX_COL2IM
  return check_launch("col2im_kernel");
}

}  // extern "C"
