// Fake-quant, EMA statistics and quantization-parameter kernels (HBM-bound).
//
// Bit-exactness with the reference's torch formulas matters here: a scale
// that differs by one ulp can flip the rounding of x/s and change LUT sums.
// The library is compiled with -ffp-contract=off, so every a*b+c below is two
// rounded operations, exactly like the separate torch ops it mirrors, and
// x/s is the correctly rounded fp32 division.

#include "atx_internal.h"

#include <algorithm>

namespace atx {

constexpr int EW = 256;   // threads per elementwise block

// torch.clamp semantics: NaN propagates (comparisons with NaN are false).
__device__ __forceinline__ float clamp_lo(float v, float lo) { return v < lo ? lo : v; }
__device__ __forceinline__ float clamp_hi(float v, float hi) { return v > hi ? hi : v; }

// ------------------------------------------- fp16 / bf16 activations
// DT: ATX_DT_F32, ATX_DT_F16 or ATX_DT_BF16.  A low-precision element is
// read as its exact fp32 value; lp_round(v) rounds an fp32 result to the
// dtype and back (round to nearest even: fp16 by the hardware conversion,
// bf16 as torch's c10::BFloat16 does, NaN to the canonical 0x7fc0), i.e.
// the value torch's elementwise kernels store after computing in fp32.
template <int DT> __device__ __forceinline__ float lp_load(const void* p, long long i) {
  if constexpr (DT == ATX_DT_F32) {
    return ((const float*)p)[i];
  } else if constexpr (DT == ATX_DT_F16) {
    return (float)__builtin_bit_cast(_Float16, ((const uint16_t*)p)[i]);
  } else {
    return __uint_as_float((unsigned)((const uint16_t*)p)[i] << 16);
  }
}
template <int DT> __device__ __forceinline__ uint16_t lp_bits(float v) {
  if constexpr (DT == ATX_DT_F16) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  } else {
    if (v != v) return 0x7fc0;
    const unsigned u = __float_as_uint(v);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
}
template <int DT> __device__ __forceinline__ float lp_round(float v) {
  if constexpr (DT == ATX_DT_F32) {
    return v;
  } else if constexpr (DT == ATX_DT_F16) {
    return (float)(_Float16)v;
  } else {
    return __uint_as_float((unsigned)lp_bits<DT>(v) << 16);
  }
}
template <int DT> __device__ __forceinline__ void lp_store(void* p, long long i, float v) {
  if constexpr (DT == ATX_DT_F32) ((float*)p)[i] = v;
  else ((uint16_t*)p)[i] = lp_bits<DT>(v);
}

// nn/quantization.py:48-52 (symmetric) and :76-80 (asymmetric);
// csrc/claude/quantization.cu:54-75.
__device__ __forceinline__ float fake_quant(float x, float s, float z, bool asym,
                                            float qmin, float qmax, bool& m) {
  float v = x / s;
  if (asym) v = v + z;
  m = (v >= qmin) && (v <= qmax);
  float r = __builtin_rintf(v);          // round half to even == torch.round
  r = clamp_lo(r, qmin);
  r = clamp_hi(r, qmax);
  return r;
}

// Byte image of a quantized value; NaN maps to 0.
__device__ __forceinline__ int to_int(float r) { return (r == r) ? (int)r : 0; }

// VEC: four elements per thread (16-byte loads, 4-byte mask / byte-image
// stores); needs n % 4 == 0 and aligned pointers.
template <bool VEC>
__global__ void fakequant_fwd_kernel(const float* __restrict__ x, long long n,
                                     const float* __restrict__ scale,
                                     const float* __restrict__ zero, float qmin,
                                     float qmax, float* __restrict__ q,
                                     uint8_t* __restrict__ mask, uint8_t* __restrict__ q8,
                                     int* __restrict__ nonneg) {
  const float s = fmaxf(scale[0], 1e-12f);
  const bool asym = zero != nullptr;
  const float z = asym ? zero[0] : 0.0f;
  const long long stride = (long long)gridDim.x * blockDim.x;
  bool neg = false;           // some quantized value < 0 (NaN counts as 0)
  if constexpr (VEC) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < (n >> 2);
         i += stride) {
      const float4 v = ((const float4*)x)[i];
      const float xv[4] = {v.x, v.y, v.z, v.w};
      float r[4];
      unsigned mk = 0, b8 = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bool m;
        r[e] = fake_quant(xv[e], s, z, asym, qmin, qmax, m);
        mk |= (m ? 1u : 0u) << (8 * e);
        b8 |= ((unsigned)to_int(r[e]) & 255u) << (8 * e);
        neg |= r[e] < 0.0f;
      }
      if (q) ((float4*)q)[i] = make_float4(r[0], r[1], r[2], r[3]);
      if (mask) ((unsigned*)mask)[i] = mk;
      if (q8) ((unsigned*)q8)[i] = b8;
    }
  } else {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) {
      bool m;
      const float r = fake_quant(x[i], s, z, asym, qmin, qmax, m);
      if (q) q[i] = r;
      if (mask) mask[i] = m;
      if (q8) q8[i] = (uint8_t)to_int(r);
      neg |= r < 0.0f;
    }
  }
  if (nonneg && neg) nonneg[0] = 0;      // benign race: every writer stores 0
}

// Fake-quant of a 1x1, stride-1, unpadded conv's input x [N,K,L] straight
// into the LUT GEMM's row-offset operand: tap k of row r = n*L + l is
// x[n][k][l], so xt[slot][r] = row_offset((to_int(q) + offset) & 255) for
// the quantized value q of x[n][operand_tap(slot, r)][l] (the index the byte
// image of fakequant_fwd_kernel gets from the im2col), and mask as
// fakequant_fwd_kernel writes it.  A thread owns one quad of rows and one
// quad of slots (blockIdx.y): it loads the 4 taps x 4 rows together (16-byte
// loads under VEC: L % 4 == 0, x 16-byte and mask 4-byte aligned), then
// writes one 8-byte xt piece per slot and one mask word per tap.  One quad
// of taps per thread keeps the grid large when N*L is small (late layers).
// Rows r >= N*L and taps k >= K hold offset 0 and write no mask.
template <bool VEC>
__global__ void __launch_bounds__(EW)
fakequant_rows_kernel(const float* __restrict__ x, int N, int K, int L,
                      const float* __restrict__ scale, const float* __restrict__ zero,
                      float qmin, float qmax, int offset, uint8_t* __restrict__ mask,
                      uint16_t* __restrict__ xt, int Rpad, int* __restrict__ upper) {
  const int q = blockIdx.x * EW + threadIdx.x;
  if (q >= (Rpad >> 2)) return;
  const float s = fmaxf(scale[0], 1e-12f);
  const bool asym = zero != nullptr;
  const float z = asym ? zero[0] : 0.0f;
  const int R = N * L;
  const int r0 = q << 2;
  long long base[4];          // x offset of tap 0 at each of the quad's rows
  unsigned valid = 0;
  if (R > 0) {
    const int rr = min(r0, R - 1);
    int n = rr / L, l = rr - n * L;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (r0 + e < R) valid |= 1u << e;
      base[e] = (long long)n * K * L + l;
      if (++l == L) { l = 0; ++n; }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) base[e] = 0;
  }
  const int k4 = blockIdx.y * 4;
  float v[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = k4 | ((q + u) & 3);          // this quad's tap of slot k4 + u
    const long long kl = (long long)min(k, K - 1) * L;
    if constexpr (VEC) {
      // L % 4 == 0: the quad is four consecutive elements of one x row,
      // wholly inside R or wholly padding
      const float4 f = (k < K && valid) ? *(const float4*)(x + base[0] + kl)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
      v[u][0] = f.x; v[u][1] = f.y; v[u][2] = f.z; v[u][3] = f.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[u][e] = (k < K && ((valid >> e) & 1u)) ? x[base[e] + kl] : 0.0f;
    }
  }
  uint16_t* dst = xt + (long long)k4 * Rpad + r0;
  bool low = false;           // some written index < 128
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = k4 | ((q + u) & 3);
    const long long kl = (long long)k * L;
    unsigned off[4], mk = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bool m;
      const float r = fake_quant(v[u][e], s, z, asym, qmin, qmax, m);
      const unsigned idx = (unsigned)(to_int(r) + offset) & 255u;
      const bool live = k < K && ((valid >> e) & 1u);
      off[e] = live ? row_offset(idx) : 0u;
      low |= live && idx < 128u;
      mk |= (m ? 1u : 0u) << (8 * e);
    }
    *(uint2*)(dst + (long long)u * Rpad) =
        make_uint2(off[0] | (off[1] << 16), off[2] | (off[3] << 16));
    if (k < K) {
      if constexpr (VEC) {
        if (valid) *(unsigned*)(mask + base[0] + kl) = mk;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((valid >> e) & 1u) mask[base[e] + kl] = (uint8_t)((mk >> (8 * e)) & 1u);
      }
    }
  }
  if (upper && low) upper[0] = 0;        // benign race: every writer stores 0
}

// gx = (mask ? go : 0) / s[c], c = (i / inner) % C.
__global__ void fakequant_bwd_kernel(const float* __restrict__ go,
                                     const uint8_t* __restrict__ mask, long long n,
                                     const float* __restrict__ scale, int C,
                                     long long inner, float* __restrict__ gx) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) {
    const int c = C == 1 ? 0 : (int)((i / inner) % C);
    const float s = fmaxf(scale[c], 1e-12f);
    gx[i] = (mask[i] ? go[i] : 0.0f) / s;
  }
}

// Per-tensor fake-quant of a low-precision x, the statements of
// nn/quantization.py:44-52 / 72-80 (the unfused path the reference takes for
// a non-fp32 x) as torch evaluates them in the input's dtype D: s =
// clamp(scale, 1e-12) in fp32; v = x / s with s first cast to D, computed in
// fp32 and rounded to D; (+ zero_point, cast to D, rounded to D); mask =
// qmin <= v <= qmax; q = clamp(round(v)) (exact in D).  q in D, mask and the
// byte image q8 (NaN -> 0) as fakequant_fwd_kernel writes them.
template <int DT>
__global__ void fakequant_fwd_lp_kernel(const void* __restrict__ x, long long n,
                                        const float* __restrict__ scale,
                                        const float* __restrict__ zero, float qmin, float qmax,
                                        void* __restrict__ q, uint8_t* __restrict__ mask,
                                        uint8_t* __restrict__ q8, int* __restrict__ nonneg) {
  const float s = lp_round<DT>(fmaxf(scale[0], 1e-12f));
  const bool asym = zero != nullptr;
  const float z = asym ? lp_round<DT>(zero[0]) : 0.0f;
  const long long stride = (long long)gridDim.x * blockDim.x;
  bool neg = false;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) {
    float v = lp_round<DT>(lp_load<DT>(x, i) / s);
    if (asym) v = lp_round<DT>(v + z);
    const bool m = (v >= qmin) && (v <= qmax);
    float r = __builtin_rintf(v);
    r = clamp_hi(clamp_lo(r, qmin), qmax);
    if (q) lp_store<DT>(q, i, r);
    if (mask) mask[i] = m;
    if (q8) q8[i] = (uint8_t)to_int(r);
    neg |= r < 0.0f;
  }
  if (nonneg && neg) nonneg[0] = 0;      // benign race: every writer stores 0
}

// grad_x = grad_output * mask.to(D) / s (nn/quantization.py:58-62) in the
// dtype D of x: the incoming gradient in GT (fp32: first rounded to D, as
// autograd casts a gradient to its input's dtype, or D itself), times the
// mask (an exact product, -0 and NaN from 0 * inf included), divided by s
// cast to D and rounded to D.
template <int GT, int DT>
__global__ void fakequant_bwd_lp_kernel(const void* __restrict__ go,
                                        const uint8_t* __restrict__ mask, long long n,
                                        const float* __restrict__ scale,
                                        void* __restrict__ gx) {
  const float s = lp_round<DT>(fmaxf(scale[0], 1e-12f));
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) {
    const float g = lp_round<DT>(lp_load<GT>(go, i));
    const float gm = g * (mask[i] ? 1.0f : 0.0f);
    lp_store<DT>(gx, i, lp_round<DT>(gm / s));
  }
}

// Weight [O, inner] per-channel fake-quant; wt is the LUT GEMM's transposed
// weight operand [inner][Opad] (columns >= O hold index 0).  A block owns a
// tile of FQ_O channels x FQ_K taps: it reads w and writes q / mask / wq
// along the taps (coalesced), stages the LUT indices in LDS and writes the
// tile's wt rows (FQ_O bytes each) as 4-byte pieces.
constexpr int FQ_O = 32, FQ_K = 64;
__global__ void __launch_bounds__(256)
fakequant_channel_kernel(const float* __restrict__ w, int O, long long inner,
                         const float* __restrict__ scale, const float* __restrict__ zero,
                         float qmin, float qmax, int offset, float* __restrict__ q,
                         uint8_t* __restrict__ mask, uint8_t* __restrict__ wq,
                         uint8_t* __restrict__ wt, int Opad) {
  __shared__ uint8_t tile[FQ_K][FQ_O + 4];
  const long long k0 = (long long)blockIdx.x * FQ_K;
  const int o0 = blockIdx.y * FQ_O;
  const bool asym = zero != nullptr;
  // quantize: thread t handles taps (t & 63) of channels o0 + (t >> 6) + 4j
  const int kl = threadIdx.x & (FQ_K - 1);
  const long long k = k0 + kl;
#pragma unroll
  for (int j = 0; j < FQ_O / 4; ++j) {
    const int ol = (threadIdx.x >> 6) + 4 * j;
    const int o = o0 + ol;
    unsigned idx = 0;
    if (o < O && k < inner) {
      const float sc = fmaxf(scale[o], 1e-12f);
      bool m;
      const long long i = (long long)o * inner + k;
      const float r = fake_quant(w[i], sc, asym ? zero[o] : 0.0f, asym, qmin, qmax, m);
      if (q) q[i] = r;
      if (mask) mask[i] = m;
      int v = to_int(r) + offset;
      v = v < 0 ? 0 : (v > 255 ? 255 : v);
      idx = (unsigned)v;
      if (wq) wq[i] = (uint8_t)idx;
    }
    tile[kl][ol] = (uint8_t)idx;
  }
  if (!wt) return;
  __syncthreads();
  // wt rows: FQ_K rows of FQ_O bytes = 512 pieces of 4 bytes
#pragma unroll
  for (int j = 0; j < (FQ_K * FQ_O / 4) / 256; ++j) {
    const int piece = threadIdx.x + 256 * j;
    const int r = piece / (FQ_O / 4), c4 = (piece % (FQ_O / 4)) * 4;
    const long long kk = k0 + r;
    if (kk < inner && o0 + c4 < Opad) {
      const unsigned v = (unsigned)tile[r][c4] | ((unsigned)tile[r][c4 + 1] << 8) |
                         ((unsigned)tile[r][c4 + 2] << 16) | ((unsigned)tile[r][c4 + 3] << 24);
      *(unsigned*)(wt + kk * Opad + o0 + c4) = v;
    }
  }
}

// ------------------------------------------------------------ reductions
// NaN-propagating max/min (torch.max / torch.amin semantics).
__device__ __forceinline__ float nmax(float a, float b) {
  return (a != a) ? a : ((b > a || b != b) ? b : a);
}
__device__ __forceinline__ float nmin(float a, float b) {
  return (a != a) ? a : ((b < a || b != b) ? b : a);
}

template <bool ABS>
__device__ __forceinline__ void block_minmax(float& mn, float& mx) {
  __shared__ float smn[EW / 64], smx[EW / 64];
  for (int off = 32; off > 0; off >>= 1) {
    mn = nmin(mn, __shfl_xor(mn, off));
    mx = nmax(mx, __shfl_xor(mx, off));
  }
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { smn[wv] = mn; smx[wv] = mx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < EW / 64; ++i) { mn = nmin(mn, smn[i]); mx = nmax(mx, smx[i]); }
  }
}

// Pass 1: per-block min / max (or |x| max) into part[2*block].  DT: the
// input's dtype (low-precision elements are exact in fp32, so the extrema
// are the dtype's own).
template <bool ABS, int DT = ATX_DT_F32>
__global__ void minmax_partial_kernel(const void* __restrict__ xv, long long n,
                                      float* __restrict__ part) {
  float mn = __builtin_inff(), mx = ABS ? 0.0f : -__builtin_inff();
  const long long stride = (long long)gridDim.x * blockDim.x;
  const long long t0 = blockIdx.x * (long long)blockDim.x + threadIdx.x;
  // 16-byte loads over the aligned body, then the remaining elements
  constexpr int PER = DT == ATX_DT_F32 ? 4 : 8;        // elements per 16 bytes
  const long long nv = ((uintptr_t)xv & 15) == 0 ? n / PER : 0;
  for (long long i = t0; i < nv; i += stride) {
    const uint4 v = ((const uint4*)xv)[i];
    const unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      float e;
      if constexpr (DT == ATX_DT_F32) {
        e = __uint_as_float(w[j]);
      } else {
        const uint16_t h = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
        e = lp_load<DT>(&h, 0);
      }
      const float u = ABS ? fabsf(e) : e;
      mn = nmin(mn, u);
      mx = nmax(mx, u);
    }
  }
  for (long long i = PER * nv + t0; i < n; i += stride) {
    const float e = lp_load<DT>(xv, i);
    const float v = ABS ? fabsf(e) : e;
    mn = nmin(mn, v);
    mx = nmax(mx, v);
  }
  block_minmax<ABS>(mn, mx);
  if (threadIdx.x == 0) { part[2 * blockIdx.x] = mn; part[2 * blockIdx.x + 1] = mx; }
}

// EMA of the statistics, applied by the final reduction block when fused.
struct EmaArgs {
  int kind;                 // 0: none, 1: int8 absmax scale, 2: uint8 min/max qparams,
                            // 3: int8 absmax scale from (min, max) plus the x >= 0 flag
  float denom, m32, om32, qmax;
  float* scale; float* zero; float* x_min; float* x_max;
  int* upper;               // kind 3: 1 when min(x) >= 0 (no NaN), else 0
  int dt;                   // kinds 1, 3: the input's dtype (ema_absmax_dt)
};
__device__ void apply_ema(const EmaArgs& e, float mn, float mx);

// Pass 2: one block folds the partials (and applies the EMA when fused).
template <bool ABS>
__global__ void minmax_final_kernel(const float* __restrict__ part, int nb,
                                    float* mn_out, float* mx_out, EmaArgs ema) {
  float mn = __builtin_inff(), mx = ABS ? 0.0f : -__builtin_inff();
  for (int i = threadIdx.x; i < nb; i += blockDim.x) {
    mn = nmin(mn, part[2 * i]);
    mx = nmax(mx, part[2 * i + 1]);
  }
  block_minmax<ABS>(mn, mx);
  if (threadIdx.x == 0) {
    if (ema.kind == 3) {
      // max |x| = max(-min x, max x) exactly (NaN propagates through both);
      // the flag holds for every x >= 0, -0 included
      ema.upper[0] = (mn >= 0.0f) ? 1 : 0;
      mx = nmax(-mn, mx);
      mn = 0.0f;
    }
    if (mn_out) *mn_out = mn;
    if (mx_out) *mx_out = mx;
    if (ema.kind) apply_ema(ema, mn, mx);
  }
}

constexpr int RED_BLOCKS = 1024;   // partial-result slots (2 floats each)

// torch on the GPU evaluates `tensor / number` (a python number) as the
// tensor times the fp32 reciprocal 1.0f / float(number), not as a division
// (its true-divide kernel's scalar path); the statistics below follow that.
__device__ __forceinline__ float div_by_number(float v, float number) {
  return v * (1.0f / number);
}

// nn/Conv2d_int8.py:144-146 — cur = stat / denom; new = m*cur + (1-m)*old.
// For an x of dtype D (fp16 / bf16) abs_max is a D scalar, so torch rounds
// cur and m * cur to D; (1 - m) * scale_x and the sum stay fp32 (a D and an
// fp32 0-dim tensor promote to fp32).
template <int DT>
__device__ __forceinline__ void ema_absmax_t(float stat, float denom, float m32, float om32,
                                             float* scale) {
  const float cur = lp_round<DT>(div_by_number(stat, denom));
  const float a = lp_round<DT>(m32 * cur);
  const float b = om32 * scale[0];
  scale[0] = a + b;
}
__device__ __forceinline__ void ema_absmax(float stat, float denom, float m32, float om32,
                                           float* scale, int dt = ATX_DT_F32) {
  if (dt == ATX_DT_F16) ema_absmax_t<ATX_DT_F16>(stat, denom, m32, om32, scale);
  else if (dt == ATX_DT_BF16) ema_absmax_t<ATX_DT_BF16>(stat, denom, m32, om32, scale);
  else ema_absmax_t<ATX_DT_F32>(stat, denom, m32, om32, scale);
}
__global__ void ema_absmax_kernel(const float* stat, float denom, float m32, float om32,
                                  float* scale, int dt) {
  ema_absmax(stat[0], denom, m32, om32, scale, dt);
}

// nn/Conv2d_uint8.py:11-23 (uint8_qparams) for one (min, max) pair.
__device__ __forceinline__ void uint8_qparams(float mn, float mx, float qmax,
                                              float& scale, float& zero) {
  mn = clamp_hi(mn, 0.0f);
  mx = clamp_lo(mx, 0.0f);
  scale = clamp_lo(div_by_number(mx - mn, qmax), 1e-12f);
  const float z = __builtin_rintf(-mn / scale);
  zero = clamp_hi(clamp_lo(z, 0.0f), qmax);
}

// nn/Conv2d_uint8.py:234-240.
__device__ __forceinline__ void ema_minmax(float mn, float mx, float m32, float om32,
                                           float qmax, float* x_min, float* x_max,
                                           float* scale, float* zero) {
  x_min[0] = m32 * mn + om32 * x_min[0];
  x_max[0] = m32 * mx + om32 * x_max[0];
  uint8_qparams(x_min[0], x_max[0], qmax, scale[0], zero[0]);
}
__global__ void ema_minmax_kernel(const float* mn, const float* mx, float m32, float om32,
                                  float qmax, float* x_min, float* x_max, float* scale,
                                  float* zero) {
  ema_minmax(mn[0], mx[0], m32, om32, qmax, x_min, x_max, scale, zero);
}

__device__ void apply_ema(const EmaArgs& e, float mn, float mx) {
  if (e.kind == 1 || e.kind == 3) ema_absmax(mx, e.denom, e.m32, e.om32, e.scale, e.dt);
  else ema_minmax(mn, mx, e.m32, e.om32, e.qmax, e.x_min, e.x_max, e.scale, e.zero);
}

// Per-channel reductions of a weight [O, inner]: one block per channel.
// mode 0: int8 absmax EMA (nn/Conv2d_int8.py:148-158)
// mode 1: int8 absmax reset (nn/Conv2d_int8.py:160-167)
// mode 2: uint8 min/max EMA + qparams (nn/Conv2d_uint8.py:242-255)
// DT: the weight's dtype.  For an fp16 / bf16 weight torch's absmax / qmax_w
// is a tensor of that dtype (rounded to it); torch.where with the fp32
// scale then promotes it back to fp32 exactly.
template <int DT>
__global__ void weight_stats_kernel(const void* __restrict__ w, long long inner, int mode,
                                    float qmax, float m32, float om32, float* scale_w,
                                    float* zero_w, float* w_min, float* w_max) {
  const int o = blockIdx.x;
  const long long base = (long long)o * inner;
  const bool absmode = mode != 2;
  float mn = __builtin_inff(), mx = absmode ? 0.0f : -__builtin_inff();
  for (long long i = threadIdx.x; i < inner; i += blockDim.x) {
    const float e = lp_load<DT>(w, base + i);
    const float v = absmode ? fabsf(e) : e;
    mn = nmin(mn, v);
    mx = nmax(mx, v);
  }
  block_minmax<false>(mn, mx);
  if (threadIdx.x != 0) return;
  if (mode == 0) {
    const float cur = (mx > 0.0f) ? lp_round<DT>(div_by_number(mx, qmax)) : scale_w[o];
    scale_w[o] = m32 * cur + om32 * scale_w[o];
  } else if (mode == 1) {
    scale_w[o] = (mx > 0.0f) ? lp_round<DT>(div_by_number(mx, qmax)) : 1.0f;
  } else {
    w_min[o] = m32 * mn + om32 * w_min[o];
    w_max[o] = m32 * mx + om32 * w_max[o];
    uint8_qparams(w_min[o], w_max[o], qmax, scale_w[o], zero_w[o]);
  }
}

// Zero-point correction and dequant of a uint8 conv's raw LUT sums, in
// place: y[n,o,l] = ((((y - zw[o]*xs[n,l]) - zx*ws[o]) + (K*zx)*zw[o]) *
// (sx*sw[o])) [+ bias[o]], the fp32 operations of nn/Conv2d_uint8.py:308-325
// in their order (xs = the taps' sum of q_x, ws[o] = sum_k q_w[o,k]).  VEC:
// L % 4 == 0, four positions of one (n, o) per thread.
template <bool VEC>
__global__ void uint8_dequant_kernel(float* __restrict__ y, long long rows, int O, int L,
                                     const float* __restrict__ xs,
                                     const float* __restrict__ ws,
                                     const float* __restrict__ zx,
                                     const float* __restrict__ zw,
                                     const float* __restrict__ sx,
                                     const float* __restrict__ sw,
                                     const float* __restrict__ bias, float K) {
  const float z = zx[0];
  const float kz = K * z;
  const float s0 = sx[0];
  const long long stride = (long long)gridDim.x * blockDim.x;
  const int W = VEC ? 4 : 1;
  const long long per_row = L / W;                      // work items per (n, o) row
  const long long total = rows * per_row;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
    const long long row = i / per_row;                  // n * O + o
    const int l = (int)(i - row * per_row) * W;
    const int o = (int)(row % O);
    const long long n = row / O;
    const float zo = zw[o], wo = z * ws[o], ko = kz * zo, so = s0 * sw[o];
    const float b = bias ? bias[o] : 0.f;
    float v[4], x[4];
    float* yp = y + row * L + l;
    const float* xp = xs + n * L + l;
    if constexpr (VEC) {
      const float4 a = *(const float4*)yp, c = *(const float4*)xp;
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      x[0] = c.x; x[1] = c.y; x[2] = c.z; x[3] = c.w;
    } else {
      v[0] = yp[0]; x[0] = xp[0];
    }
#pragma unroll
    for (int e = 0; e < W; ++e) v[e] = u8_dequant(v[e], x[e], zo, wo, ko, so, bias, b);
    if constexpr (VEC) *(float4*)yp = make_float4(v[0], v[1], v[2], v[3]);
    else yp[0] = v[0];
  }
}

}  // namespace atx

using namespace atx;

extern "C" {

int atx_fakequant_fwd(const float* x, long long n, const float* scale, const float* zero,
                      int qmin, int qmax, float* q, uint8_t* mask, void* q8, int* nonneg,
                      hipStream_t stream) {
  ATX_REQUIRE(n >= 0, "atx_fakequant_fwd: negative size");
  ATX_REQUIRE(qmin < qmax, "qmin must be < qmax, got [%d, %d]", qmin, qmax);
  if (n == 0) return ATX_OK;
  ATX_REQUIRE(x && scale, "atx_fakequant_fwd: null pointer");
  const bool vec = n % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 15) == 0 &&
                   ((uintptr_t)mask & 3) == 0 && ((uintptr_t)q8 & 3) == 0;
  if (vec)
    hipLaunchKernelGGL(fakequant_fwd_kernel<true>, dim3(elem_grid(n / 4, EW)), dim3(EW), 0,
                       stream, x, n, scale, zero, (float)qmin, (float)qmax, q, mask,
                       (uint8_t*)q8, nonneg);
  else
    hipLaunchKernelGGL(fakequant_fwd_kernel<false>, dim3(elem_grid(n, EW)), dim3(EW), 0,
                       stream, x, n, scale, zero, (float)qmin, (float)qmax, q, mask,
                       (uint8_t*)q8, nonneg);
  return check_launch("fakequant_fwd_kernel");
}

int atx_fakequant_rows(const float* x, int N, int K, int L, const float* scale,
                       const float* zero, int qmin, int qmax, int offset, uint8_t* mask,
                       uint16_t* xt, int Rpad, int* upper, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0, "atx_fakequant_rows: negative size");
  ATX_REQUIRE(qmin < qmax, "qmin must be < qmax, got [%d, %d]", qmin, qmax);
  ATX_REQUIRE(offset == 0 || offset == 128, "atx_fakequant_rows: offset must be 0 or 128");
  ATX_REQUIRE(Rpad >= (long long)N * L && Rpad % ATX_ROW_TILE == 0,
              "atx_fakequant_rows: Rpad must be a multiple of %d covering N*L", ATX_ROW_TILE);
  if ((long long)K * Rpad == 0) return ATX_OK;
  // an empty x (N*L == 0) only writes the zero padding rows
  ATX_REQUIRE(xt && scale && ((long long)N * L == 0 || (x && mask)),
              "atx_fakequant_rows: null pointer");
  ATX_REQUIRE(operand_rows(K) / 4 <= 65535, "atx_fakequant_rows: K too large");
  const dim3 grid((unsigned)cdiv(Rpad / 4, EW), (unsigned)(operand_rows(K) / 4));
  const bool vec = L % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)mask & 3) == 0;
  if (vec)
    hipLaunchKernelGGL(fakequant_rows_kernel<true>, grid, dim3(EW), 0, stream, x, N, K, L,
                       scale, zero, (float)qmin, (float)qmax, offset, mask, xt, Rpad, upper);
  else
    hipLaunchKernelGGL(fakequant_rows_kernel<false>, grid, dim3(EW), 0, stream, x, N, K, L,
                       scale, zero, (float)qmin, (float)qmax, offset, mask, xt, Rpad, upper);
  return check_launch("fakequant_rows_kernel");
}

int atx_fakequant_bwd(const float* go, const uint8_t* mask, long long n, const float* scale,
                      int C, long long inner, float* gx, hipStream_t stream) {
  ATX_REQUIRE(n >= 0 && C >= 1 && inner >= 1, "atx_fakequant_bwd: bad size");
  if (n == 0) return ATX_OK;
  ATX_REQUIRE(go && mask && scale && gx, "atx_fakequant_bwd: null pointer");
  hipLaunchKernelGGL(fakequant_bwd_kernel, dim3(elem_grid(n, EW)), dim3(EW), 0, stream, go,
                     mask, n, scale, C, inner, gx);
  return check_launch("fakequant_bwd_kernel");
}

int atx_fakequant_channel_fwd(const float* w, int O, long long inner, const float* scale,
                              const float* zero, int qmin, int qmax, int offset, float* q,
                              uint8_t* mask, uint8_t* wq, uint8_t* wt, int Opad,
                              hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && inner >= 0, "atx_fakequant_channel_fwd: negative size");
  ATX_REQUIRE(qmin < qmax, "qmin must be < qmax, got [%d, %d]", qmin, qmax);
  ATX_REQUIRE(!wt || (Opad >= O && Opad % ATX_COL_TILE == 0),
              "atx_fakequant_channel_fwd: bad Opad %d", Opad);
  const long long cols = wt ? Opad : O;
  if (inner * cols == 0) return ATX_OK;
  ATX_REQUIRE(w && scale, "atx_fakequant_channel_fwd: null pointer");
  ATX_REQUIRE(cdiv(inner, FQ_K) <= 0x7fffffffLL && cdiv(cols, FQ_O) <= 65535,
              "atx_fakequant_channel_fwd: weight too large");
  ATX_REQUIRE(((uintptr_t)wt & 3) == 0, "atx_fakequant_channel_fwd: wt must be 4-byte aligned");
  const dim3 grid((unsigned)cdiv(inner, FQ_K), (unsigned)cdiv(cols, FQ_O));
  hipLaunchKernelGGL(fakequant_channel_kernel, grid, dim3(256), 0, stream, w, O, inner, scale,
                     zero, (float)qmin, (float)qmax, offset, q, mask, wq, wt, (int)cols);
  return check_launch("fakequant_channel_kernel");
}

static int minmax_impl(const void* x, long long n, unsigned int* ws, float* mn_out,
                       float* mx_out, bool absmode, hipStream_t stream,
                       EmaArgs ema = EmaArgs{}, int dt = ATX_DT_F32) {
  ATX_REQUIRE(n > 0, "min/max of an empty tensor is undefined");
  ATX_REQUIRE(x && ws, "minmax: null pointer");
  ATX_REQUIRE(dt == ATX_DT_F32 || dt == ATX_DT_F16 || dt == ATX_DT_BF16,
              "minmax: bad dtype %d", dt);
  const int nb = elem_grid(n, EW, RED_BLOCKS);
  float* part = (float*)ws;
  ema.dt = dt;
#define ATX_MM(A, D) \
  hipLaunchKernelGGL((minmax_partial_kernel<A, D>), dim3(nb), dim3(EW), 0, stream, x, n, part)
  if (dt == ATX_DT_F16) { if (absmode) ATX_MM(true, ATX_DT_F16); else ATX_MM(false, ATX_DT_F16); }
  else if (dt == ATX_DT_BF16) { if (absmode) ATX_MM(true, ATX_DT_BF16); else ATX_MM(false, ATX_DT_BF16); }
  else { if (absmode) ATX_MM(true, ATX_DT_F32); else ATX_MM(false, ATX_DT_F32); }
#undef ATX_MM
  int rc = check_launch("minmax_partial_kernel");
  if (rc) return rc;
  if (absmode)
    hipLaunchKernelGGL(minmax_final_kernel<true>, dim3(1), dim3(EW), 0, stream, part, nb,
                       mn_out, mx_out, ema);
  else
    hipLaunchKernelGGL(minmax_final_kernel<false>, dim3(1), dim3(EW), 0, stream, part, nb,
                       mn_out, mx_out, ema);
  return check_launch("minmax_final_kernel");
}

long long atx_reduce_workspace_bytes(void) { return (long long)RED_BLOCKS * 2 * 4; }

int atx_absmax(const float* x, long long n, unsigned int* ws, float* stat_out,
               hipStream_t stream) {
  ATX_REQUIRE(stat_out, "atx_absmax: null output");
  return minmax_impl(x, n, ws, nullptr, stat_out, true, stream);
}

int atx_minmax(const float* x, long long n, unsigned int* ws, float* mn_out, float* mx_out,
               hipStream_t stream) {
  ATX_REQUIRE(mn_out && mx_out, "atx_minmax: null output");
  return minmax_impl(x, n, ws, mn_out, mx_out, false, stream);
}

int atx_absmax_ema(const float* x, long long n, unsigned int* ws, float* stat_out,
                   float denom, float m32, float om32, float* scale, hipStream_t stream) {
  ATX_REQUIRE(stat_out && scale, "atx_absmax_ema: null output");
  EmaArgs e{};
  e.kind = 1; e.denom = denom; e.m32 = m32; e.om32 = om32; e.scale = scale;
  return minmax_impl(x, n, ws, nullptr, stat_out, true, stream, e);
}

int atx_absmax_ema_upper(const float* x, long long n, unsigned int* ws, float* stat_out,
                         float denom, float m32, float om32, float* scale, int* upper,
                         hipStream_t stream) {
  ATX_REQUIRE(stat_out && scale && upper, "atx_absmax_ema_upper: null output");
  EmaArgs e{};
  e.kind = 3; e.denom = denom; e.m32 = m32; e.om32 = om32; e.scale = scale; e.upper = upper;
  return minmax_impl(x, n, ws, nullptr, stat_out, false, stream, e);
}

int atx_minmax_ema(const float* x, long long n, unsigned int* ws, float* mn_out,
                   float* mx_out, float m32, float om32, int qmax, float* x_min, float* x_max,
                   float* scale, float* zero, hipStream_t stream) {
  ATX_REQUIRE(mn_out && mx_out && x_min && x_max && scale && zero, "atx_minmax_ema: null");
  EmaArgs e{};
  e.kind = 2; e.m32 = m32; e.om32 = om32; e.qmax = (float)qmax;
  e.scale = scale; e.zero = zero; e.x_min = x_min; e.x_max = x_max;
  return minmax_impl(x, n, ws, mn_out, mx_out, false, stream, e);
}

int atx_ema_absmax_apply(const float* stat, float denom, float m32, float om32, float* scale,
                         hipStream_t stream) {
  ATX_REQUIRE(stat && scale, "atx_ema_absmax_apply: null pointer");
  hipLaunchKernelGGL(ema_absmax_kernel, dim3(1), dim3(1), 0, stream, stat, denom, m32, om32,
                     scale, (int)ATX_DT_F32);
  return check_launch("ema_absmax_kernel");
}

int atx_absmax_dt(const void* x, int dtype, long long n, unsigned int* ws, float* stat_out,
                  hipStream_t stream) {
  ATX_REQUIRE(stat_out, "atx_absmax_dt: null output");
  return minmax_impl(x, n, ws, nullptr, stat_out, true, stream, EmaArgs{}, dtype);
}

int atx_ema_absmax_apply_dt(const float* stat, int dtype, float denom, float m32, float om32,
                            float* scale, hipStream_t stream) {
  ATX_REQUIRE(stat && scale, "atx_ema_absmax_apply_dt: null pointer");
  ATX_REQUIRE(dtype == ATX_DT_F32 || dtype == ATX_DT_F16 || dtype == ATX_DT_BF16,
              "atx_ema_absmax_apply_dt: bad dtype %d", dtype);
  hipLaunchKernelGGL(ema_absmax_kernel, dim3(1), dim3(1), 0, stream, stat, denom, m32, om32,
                     scale, dtype);
  return check_launch("ema_absmax_kernel");
}

int atx_absmax_ema_upper_dt(const void* x, int dtype, long long n, unsigned int* ws,
                            float* stat_out, float denom, float m32, float om32, float* scale,
                            int* upper, hipStream_t stream) {
  ATX_REQUIRE(stat_out && scale && upper, "atx_absmax_ema_upper_dt: null output");
  EmaArgs e{};
  e.kind = 3; e.denom = denom; e.m32 = m32; e.om32 = om32; e.scale = scale; e.upper = upper;
  return minmax_impl(x, n, ws, nullptr, stat_out, false, stream, e, dtype);
}

int atx_fakequant_fwd_dt(const void* x, int dtype, long long n, const float* scale,
                         const float* zero, int qmin, int qmax, void* q, uint8_t* mask,
                         void* q8, int* nonneg, hipStream_t stream) {
  ATX_REQUIRE(n >= 0, "atx_fakequant_fwd_dt: negative size");
  ATX_REQUIRE(qmin < qmax, "qmin must be < qmax, got [%d, %d]", qmin, qmax);
  ATX_REQUIRE(dtype == ATX_DT_F16 || dtype == ATX_DT_BF16,
              "atx_fakequant_fwd_dt: dtype must be ATX_DT_F16 or ATX_DT_BF16, got %d", dtype);
  if (n == 0) return ATX_OK;
  ATX_REQUIRE(x && scale, "atx_fakequant_fwd_dt: null pointer");
  const dim3 grid(elem_grid(n, EW));
  if (dtype == ATX_DT_F16)
    hipLaunchKernelGGL(fakequant_fwd_lp_kernel<ATX_DT_F16>, grid, dim3(EW), 0, stream, x, n,
                       scale, zero, (float)qmin, (float)qmax, q, mask, (uint8_t*)q8, nonneg);
  else
    hipLaunchKernelGGL(fakequant_fwd_lp_kernel<ATX_DT_BF16>, grid, dim3(EW), 0, stream, x, n,
                       scale, zero, (float)qmin, (float)qmax, q, mask, (uint8_t*)q8, nonneg);
  return check_launch("fakequant_fwd_lp_kernel");
}

int atx_fakequant_bwd_dt(const void* go, int go_dtype, const uint8_t* mask, long long n,
                         const float* scale, int dtype, void* gx, hipStream_t stream) {
  ATX_REQUIRE(n >= 0, "atx_fakequant_bwd_dt: negative size");
  ATX_REQUIRE(dtype == ATX_DT_F16 || dtype == ATX_DT_BF16,
              "atx_fakequant_bwd_dt: dtype must be ATX_DT_F16 or ATX_DT_BF16, got %d", dtype);
  ATX_REQUIRE(go_dtype == ATX_DT_F32 || go_dtype == dtype,
              "atx_fakequant_bwd_dt: go must be fp32 or the dtype of x");
  if (n == 0) return ATX_OK;
  ATX_REQUIRE(go && mask && scale && gx, "atx_fakequant_bwd_dt: null pointer");
  const dim3 grid(elem_grid(n, EW));
#define ATX_FQB(G, D) \
  hipLaunchKernelGGL((fakequant_bwd_lp_kernel<G, D>), grid, dim3(EW), 0, stream, go, mask, n, \
                     scale, gx)
  if (dtype == ATX_DT_F16) {
    if (go_dtype == ATX_DT_F32) ATX_FQB(ATX_DT_F32, ATX_DT_F16); else ATX_FQB(ATX_DT_F16, ATX_DT_F16);
  } else {
    if (go_dtype == ATX_DT_F32) ATX_FQB(ATX_DT_F32, ATX_DT_BF16); else ATX_FQB(ATX_DT_BF16, ATX_DT_BF16);
  }
#undef ATX_FQB
  return check_launch("fakequant_bwd_lp_kernel");
}

int atx_ema_minmax_apply(const float* mn, const float* mx, float m32, float om32, int qmax,
                         float* x_min, float* x_max, float* scale, float* zero,
                         hipStream_t stream) {
  ATX_REQUIRE(mn && mx && x_min && x_max && scale && zero, "atx_ema_minmax_apply: null");
  hipLaunchKernelGGL(ema_minmax_kernel, dim3(1), dim3(1), 0, stream, mn, mx, m32, om32,
                     (float)qmax, x_min, x_max, scale, zero);
  return check_launch("ema_minmax_kernel");
}

int atx_weight_scale_ema_dt(const void* w, int dtype, int O, long long inner, float qmax_w,
                            float m32, float om32, int reset, float* scale_w,
                            hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && inner > 0, "atx_weight_scale_ema: bad size");
  ATX_REQUIRE(dtype == ATX_DT_F32 || dtype == ATX_DT_F16 || dtype == ATX_DT_BF16,
              "atx_weight_scale_ema: bad dtype %d", dtype);
  if (O == 0) return ATX_OK;
  ATX_REQUIRE(w && scale_w, "atx_weight_scale_ema: null pointer");
#define ATX_WS(D)                                                                         \
  hipLaunchKernelGGL(weight_stats_kernel<D>, dim3(O), dim3(EW), 0, stream, w, inner,     \
                     reset ? 1 : 0, qmax_w, m32, om32, scale_w, (float*)nullptr,          \
                     (float*)nullptr, (float*)nullptr)
  if (dtype == ATX_DT_F16) ATX_WS(ATX_DT_F16);
  else if (dtype == ATX_DT_BF16) ATX_WS(ATX_DT_BF16);
  else ATX_WS(ATX_DT_F32);
#undef ATX_WS
  return check_launch("weight_stats_kernel");
}

int atx_weight_scale_ema(const float* w, int O, long long inner, float qmax_w, float m32,
                         float om32, int reset, float* scale_w, hipStream_t stream) {
  return atx_weight_scale_ema_dt(w, ATX_DT_F32, O, inner, qmax_w, m32, om32, reset, scale_w,
                                 stream);
}

int atx_weight_minmax_ema(const float* w, int O, long long inner, float m32, float om32,
                          int qmax, float* w_min, float* w_max, float* scale_w, float* zero_w,
                          hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && inner > 0, "atx_weight_minmax_ema: bad size");
  if (O == 0) return ATX_OK;
  ATX_REQUIRE(w && w_min && w_max && scale_w && zero_w, "atx_weight_minmax_ema: null");
  hipLaunchKernelGGL(weight_stats_kernel<ATX_DT_F32>, dim3(O), dim3(EW), 0, stream, w, inner, 2,
                     (float)qmax, m32, om32, scale_w, zero_w, w_min, w_max);
  return check_launch("weight_stats_kernel");
}

int atx_uint8_dequant(float* y, int N, int O, int L, const float* xsum, const float* wsum,
                      const float* zero_x, const float* zero_w, const float* scale_x,
                      const float* scale_w, const float* bias, int K, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && O >= 0 && L >= 0 && K >= 0, "atx_uint8_dequant: negative size");
  const long long rows = (long long)N * O;
  if (rows * L == 0) return ATX_OK;
  ATX_REQUIRE(y && xsum && wsum && zero_x && zero_w && scale_x && scale_w,
              "atx_uint8_dequant: null pointer");
  const bool vec = L % 4 == 0 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)xsum & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(uint8_dequant_kernel<true>, dim3(elem_grid(rows * L / 4, EW)), dim3(EW),
                       0, stream, y, rows, O, L, xsum, wsum, zero_x, zero_w, scale_x, scale_w,
                       bias, (float)K);
  else
    hipLaunchKernelGGL(uint8_dequant_kernel<false>, dim3(elem_grid(rows * L, EW)), dim3(EW),
                       0, stream, y, rows, O, L, xsum, wsum, zero_x, zero_w, scale_x, scale_w,
                       bias, (float)K);
  return check_launch("uint8_dequant_kernel");
}

}  // extern "C"
