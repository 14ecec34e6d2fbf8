// Matrix-core (MFMA) GEMMs for the STE / LRE backward of the LUT conv.
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
// Two engines over BM x BN block tiles (64 or 128 each), 32-deep k-tiles and
// 256 threads as 2 x 2 waves:
// - split-bf16 (the layer paths): fp32 operands split exactly into three
//   bf16 parts and multiplied on v_mfma_f32_16x16x32_bf16 as the six part
//   products of order <= 2 (three when a table is bf16 already); see the
//   "split-bf16 operand planes" section below.  Backward-weight, the
//   backward-data GEMM of atx_conv_bwd_data (its A operand from bf16 weight
//   planes prepared per call) and the implicit backward-data GEMM.
// - fp32 (v_mfma_f32_16x16x4f32, plain fp32 products): the backward-data
//   GEMM of atx_conv_bwd_data_col (no workspace for the planes) and layers
//   whose go spans exceed the split path's 32-bit buffer offsets.  The
//   256-entry table lives in LDS; operand tiles go HBM -> registers while
//   the previous tile is multiplied, then through the table into a second
//   LDS buffer ([BK][B + 16], bank 16k + i: conflict-free MFMA reads); one
//   barrier per k-tile.
// The backward-data GEMMs fold the batch into their columns (c = n*L + l),
// so small images waste no tile width.

#include "atx_internal.h"
#include "atx_tiles.h"

#include <algorithm>
#include <type_traits>

namespace atx {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BK = 32;          // contraction depth of one k-tile
constexpr int GT = 256;         // threads per block (2 x 2 waves)

template <int B> struct KMajor {          // [BK][B + 16]: bank(k, i) = 16k + i
  static constexpr int LD = B + 16;
  static constexpr int SIZE = BK * LD;
  __device__ static int at(int m, int k) { return k * LD + m; }
};

// ------------------------------------------------ split-bf16 operand planes
// gfx950's bf16 matrix cores (v_mfma_f32_16x16x32_bf16: a 16 x 16 x 32 block
// in 16 cycles) do 16 times the products per cycle of its fp32 ones
// (v_mfma_f32_16x16x4f32: 16 x 16 x 4 in 32).  An fp32 value a splits exactly
// into three bf16 parts a = ah + am + al by truncation: ah is a with its low
// 16 bits cleared, r = a - ah is exact in fp32 with at most 16 significant
// bits, am is r truncated the same way and al = r - am has at most 8.  The
// product a*b is taken as the six part products of order <= 2,
//   ah*bh + ah*bm + am*bh + ah*bl + am*bm + al*bh,
// each exact in fp32 (8 x 8 significant bits), summed in fp32.  The dropped
// products am*bl + al*bm + al*bl stay below 2^-20 |a b| (|am| < 2^-7 |a|,
// |al| < 2^-14 |a|), on average about 2^-23 |a b|, the size of an fp32
// product's own rounding.  An operand whose values are bf16 already (the
// STE's quantized integers, or any table whose m and l parts are all zero)
// has only its h part: three products, each exact, instead of six.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Which part products a tile multiply takes.
enum PartProducts { PROD6 = 0, A_EXACT = 1, B_EXACT = 2 };

// Operand tile of B rows x BK contraction elements as three bf16 planes
// (h, m, l) of B x 64 bytes.  Row r is stored at s = r ^ ((r >> 2) & 1) and
// its four 16-byte units (8 contraction elements each) are XOR-swizzled by
// (s >> 1) & 3: the MFMA fragment reads (8 lanes = rows 0..7 of one unit)
// and the loaders' 8-byte stores (16 lanes = two rows r, r + 1 or r, r + 4,
// eight 8-byte groups each) are then bank-conflict-free.
template <int B> struct Planes {
  static constexpr int PLANE = B * 64;
  static constexpr int SIZE = 3 * PLANE;
  // byte offset of contraction elements k..k+3 (k % 4 == 0) of row r
  __device__ static int at(int r, int k) {
    const int s = r ^ ((r >> 2) & 1);
    return s * 64 + ((((k >> 3) ^ (s >> 1)) & 3) << 4) + ((k & 4) << 1);
  }
};

// Parts of four consecutive contraction elements, two bf16 per dword (the
// lower element in the low half): P[0] = h, P[1] = m, P[2] = l.
template <bool FULL>
__device__ __forceinline__ void split4(const float (&v)[4], uint2 (&P)[3]) {
  unsigned h[4], m[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = __float_as_uint(v[e]);
    if constexpr (FULL) {
      const float r = bf16_rest(v[e]);
      m[e] = __float_as_uint(r);
      l[e] = __float_as_uint(r - __uint_as_float(m[e] & 0xffff0000u));
    }
  }
  P[0] = make_uint2(__builtin_amdgcn_perm(h[1], h[0], 0x07060302u),
                    __builtin_amdgcn_perm(h[3], h[2], 0x07060302u));
  if constexpr (FULL) {
    P[1] = make_uint2(__builtin_amdgcn_perm(m[1], m[0], 0x07060302u),
                      __builtin_amdgcn_perm(m[3], m[2], 0x07060302u));
    P[2] = make_uint2(__builtin_amdgcn_perm(l[1], l[0], 0x07060302u),
                      __builtin_amdgcn_perm(l[3], l[2], 0x07060302u));
  }
}

// Split table: entry i = (h | m << 16, l) of tab[i]; entry 256 is zero (the
// index of invalid elements).  Returns whether every entry is bf16 exactly
// (all m and l parts zero).  Needs GT == 256 threads; ends with a barrier.
__device__ __forceinline__ bool split_table(uint2* stab, const float* tab, int t) {
  const float v = tab[t];
  const unsigned u = __float_as_uint(v);
  const float r = bf16_rest(v);
  const unsigned ru = __float_as_uint(r);
  const unsigned lo = __float_as_uint(r - __uint_as_float(ru & 0xffff0000u));
  stab[t] = make_uint2((u >> 16) | (ru & 0xffff0000u), lo >> 16);
  if (t == 0) stab[256] = make_uint2(0u, 0u);
  return __syncthreads_or(r != 0.0f) == 0;
}

// Whether every entry of a 256-entry table is bf16 exactly (GT == 256
// threads; ends with a barrier).
__device__ __forceinline__ bool table_exact(const float* tab, int t) {
  const float v = tab[t];
  return __syncthreads_or(bf16_rest(v) != 0.0f) == 0;
}

// Parts of four table entries (indices into a split table) in split4's order.
template <bool FULL>
__device__ __forceinline__ void lookup4(const uint2* stab, const unsigned (&idx)[4],
                                        uint2 (&P)[3]) {
  uint2 e[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) e[i] = stab[idx[i]];
  P[0] = make_uint2(__builtin_amdgcn_perm(e[1].x, e[0].x, 0x05040100u),
                    __builtin_amdgcn_perm(e[3].x, e[2].x, 0x05040100u));
  if constexpr (FULL) {
    P[1] = make_uint2(__builtin_amdgcn_perm(e[1].x, e[0].x, 0x07060302u),
                      __builtin_amdgcn_perm(e[3].x, e[2].x, 0x07060302u));
    P[2] = make_uint2(__builtin_amdgcn_perm(e[1].y, e[0].y, 0x05040100u),
                      __builtin_amdgcn_perm(e[3].y, e[2].y, 0x05040100u));
  }
}

template <int B, bool FULL>
__device__ __forceinline__ void put_parts(char* s, int r, int k, const uint2 (&P)[3]) {
  const int off = Planes<B>::at(r, k);
  *(uint2*)(s + off) = P[0];
  if constexpr (FULL) {
    *(uint2*)(s + Planes<B>::PLANE + off) = P[1];
    *(uint2*)(s + 2 * Planes<B>::PLANE + off) = P[2];
  }
}

// Index of an image element (int8: v + 128, uint8: v, fp32: quant_index).
template <typename T> __device__ __forceinline__ unsigned img_index(unsigned raw, int offset);
template <> __device__ __forceinline__ unsigned img_index<int8_t>(unsigned raw, int) {
  return (raw + 128u) & 255u;
}
template <> __device__ __forceinline__ unsigned img_index<uint8_t>(unsigned raw, int) {
  return raw & 255u;
}
template <> __device__ __forceinline__ unsigned img_index<float>(unsigned raw, int offset) {
  return quant_index(__uint_as_float(raw), offset);
}

// ------------------------------------------------------------- operand loaders
// Each loader owns a BK x B slice of one operand: fetch() issues the global
// loads of k-tile p0 into registers, stash() maps them through the LDS table
// (if any) and stores them into an LDS tile.  fetch() has no branches: an
// element outside the operand loads element 0 instead and its validity bit
// zeroes it in stash(), so the compiler never waits for a load before the
// MFMAs that follow.  VEC: the operand's quads are 16-byte (4-byte for
// bytes) aligned and never straddle a row, so one vector load covers them.

// Backward-data A: A(m = k, p = o) = tx[wq[o*K + k]], KMajor.
template <int B, bool VEC> struct DataA {
  using Lay = KMajor<B>;
  static constexpr int QPR = B / 4, NQ = BK * B / (4 * GT), PSTEP = GT / QPR;
  const uint8_t* wq; int K;
  int mq, pr, gm;
  unsigned raw[NQ], ok;
  __device__ void init(int t, int m0) {
    mq = (t % QPR) * 4; pr = t / QPR; gm = m0 + mq;
  }
  __device__ void fetch(int p0, int pe) {
    ok = 0;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int p = p0 + pr + i * PSTEP;
      const long long row = (long long)p * K;
      if constexpr (VEC) {
        const bool v = p < pe && gm < K;
        raw[i] = *(const unsigned*)(wq + (v ? row + gm : 0));
        ok |= (v ? 15u : 0u) << (4 * i);
      } else {
        raw[i] = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool v = p < pe && gm + e < K;
          raw[i] |= (unsigned)wq[v ? row + gm + e : 0] << (8 * e);
          ok |= (v ? 1u : 0u) << (4 * i + e);
        }
      }
    }
  }
  __device__ void stash(float* s, const float* tab) const {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      floatx4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = tab[(raw[i] >> (8 * e)) & 255u];
        v[e] = (ok >> (4 * i + e)) & 1u ? x : 0.0f;
      }
      *(floatx4*)&s[Lay::at(mq, pr + i * PSTEP)] = v;
    }
  }
  __device__ void advance() {}
};

// Backward-data B: B(p = o, j = c) = go[n][o][l] (* sx * sw[o] when SCALED)
// with c = n*L + l, KMajor.  The scale product is rounded to fp32 first and
// then applied, the order of the layer's `y * (scale_x * scale_w)`.
template <int B, bool VEC, bool SCALED> struct DataB {
  using Lay = KMajor<B>;
  static constexpr int QPR = B / 4, NQ = BK * B / (4 * GT), PSTEP = GT / QPR;
  const float* go; int O, L, NL;
  const float* sx; const float* sw;
  int jq, pr;
  float sx0;
  long long base[4];        // go offset of column c + e at o = 0 (-1: no column)
  floatx4 raw[NQ];
  float sc[NQ];
  unsigned ok;
  __device__ void init(int t, int n0) {
    jq = (t % QPR) * 4; pr = t / QPR;
    if constexpr (SCALED) sx0 = sx[0];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = n0 + jq + e;
      if (c < NL) {
        const int n = c / L;
        base[e] = (long long)n * O * L + (c - n * L);
      } else {
        base[e] = -1;
      }
    }
  }
  __device__ void fetch(int p0, int pe) {
    ok = 0;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int o = p0 + pr + i * PSTEP;
      const long long ol = (long long)o * L;
      if constexpr (SCALED) sc[i] = sw[o < pe ? o : 0];
      if constexpr (VEC) {
        const bool v = o < pe && base[0] >= 0;
        raw[i] = *(const floatx4*)(go + (v ? base[0] + ol : 0));
        ok |= (v ? 15u : 0u) << (4 * i);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool v = o < pe && base[e] >= 0;
          raw[i][e] = go[v ? base[e] + ol : 0];
          ok |= (v ? 1u : 0u) << (4 * i + e);
        }
      }
    }
  }
  __device__ void stash(float* s, const float*) const {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      floatx4 v;
      float f = 1.0f;
      if constexpr (SCALED) f = sx0 * sc[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = SCALED ? raw[i][e] * f : raw[i][e];
        v[e] = (ok >> (4 * i + e)) & 1u ? x : 0.0f;
      }
      *(floatx4*)&s[Lay::at(jq, pr + i * PSTEP)] = v;
    }
  }
  __device__ void advance() {}
};

// Implicit backward-data GEMM of a stride-1 conv (no col buffer, no fold):
//   gx[n,c,h,w] = sum over p = t*O + o (t = i*KW + j) of
//                 tx[wq[o][c*KK + t]] * go'[n, o, h + PH - i*DH, w + PW - j*DW]
// (out-of-range go positions contribute 0).  With O % BK == 0 every k-tile
// has one tap t, so its spatial shift is uniform over the tile.

// A(m = c, p) = tx[wq[o*K + c*KK + t]], KMajor (quads of four channels).
template <int B> struct DgradA {
  using Lay = KMajor<B>;
  static constexpr int QPR = B / 4, NQ = BK * B / (4 * GT), PSTEP = GT / QPR;
  const uint8_t* wq; int K, KK, C, O;
  int mq, pr, gm;
  unsigned raw[NQ], ok;
  __device__ void init(int t, int m0) { mq = (t % QPR) * 4; pr = t / QPR; gm = m0 + mq; }
  __device__ void fetch(int p0, int pe) {
    const int tap = p0 / O;                   // uniform over the k-tile
    const int o0 = p0 - tap * O;
    ok = 0;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int o = o0 + pr + i * PSTEP;
      const bool pv = p0 + pr + i * PSTEP < pe;
      raw[i] = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool v = pv && gm + e < C;
        raw[i] |= (unsigned)wq[v ? (long long)o * K + (long long)(gm + e) * KK + tap : 0]
                  << (8 * e);
        ok |= (v ? 1u : 0u) << (4 * i + e);
      }
    }
  }
  __device__ void stash(float* s, const float* tab) const {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      floatx4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = tab[(raw[i] >> (8 * e)) & 255u];
        v[e] = (ok >> (4 * i + e)) & 1u ? x : 0.0f;
      }
      *(floatx4*)&s[Lay::at(mq, pr + i * PSTEP)] = v;
    }
  }
  __device__ void advance() {}
};

// B(p, col = (n, h, w)) = go'[n, o, h + PH - i*DH, w + PW - j*DW], KMajor
// (quads of four pixels); go' = go * fp32(sx * sw[o]) when SCALED.
template <int B, bool SCALED> struct DgradB {
  using Lay = KMajor<B>;
  static constexpr int QPR = B / 4, NQ = BK * B / (4 * GT), PSTEP = GT / QPR;
  const float* go; atx_conv_geom g; int O, NHW;
  const float* sx; const float* sw;
  int jq, pr;
  float sx0;
  long long nb[4];          // go offset of image n_e (o = 0, h = w = 0); -1: no pixel
  int hh[4], ww[4];         // pixel coordinates
  floatx4 raw[NQ];
  float sc[NQ];
  unsigned ok;
  __device__ void init(int t, int n0) {
    jq = (t % QPR) * 4; pr = t / QPR;
    if constexpr (SCALED) sx0 = sx[0];
    const int HW = g.H * g.W;
    const long long OHW = (long long)g.OH * g.OW;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = n0 + jq + e;
      if (c < NHW) {
        const int n = c / HW, hw = c - n * HW;
        hh[e] = hw / g.W;
        ww[e] = hw - hh[e] * g.W;
        nb[e] = (long long)n * O * OHW;
      } else {
        nb[e] = -1; hh[e] = ww[e] = 0;
      }
    }
  }
  __device__ void fetch(int p0, int pe) {
    const int tap = p0 / O;                   // uniform over the k-tile
    const int o0 = p0 - tap * O;
    const int ki = tap / g.KW, kj = tap - ki * g.KW;
    const int dh0 = g.PH - ki * g.DH, dw0 = g.PW - kj * g.DW;
    const long long OHW = (long long)g.OH * g.OW;
    long long off[4];
    bool pv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ih = hh[e] + dh0, iw = ww[e] + dw0;
      pv[e] = nb[e] >= 0 && (unsigned)ih < (unsigned)g.OH && (unsigned)iw < (unsigned)g.OW;
      off[e] = nb[e] + (long long)ih * g.OW + iw;
    }
    ok = 0;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int o = o0 + pr + i * PSTEP;
      const bool rv = p0 + pr + i * PSTEP < pe;
      if constexpr (SCALED) sc[i] = sw[rv ? o : 0];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool v = rv && pv[e];
        raw[i][e] = go[v ? off[e] + (long long)o * OHW : 0];
        ok |= (v ? 1u : 0u) << (4 * i + e);
      }
    }
  }
  __device__ void stash(float* s, const float*) const {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      floatx4 v;
      float f = 1.0f;
      if constexpr (SCALED) f = sx0 * sc[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = SCALED ? raw[i][e] * f : raw[i][e];
        v[e] = (ok >> (4 * i + e)) & 1u ? x : 0.0f;
      }
      *(floatx4*)&s[Lay::at(jq, pr + i * PSTEP)] = v;
    }
  }
  __device__ void advance() {}
};

// Rows r = n*L + l of the weight GEMM's contraction, tracked incrementally:
// the thread's quad starts at r = p0 + pq and moves by BK per k-tile.
struct RowCursor {
  int n, l;
  __device__ void start(int r, int L) { n = r / L; l = r - n * L; }
  __device__ void step(int d, int L) {
    l += d;
    while (l >= L) { l -= L; ++n; }
  }
};

// Backward-weight A: A(m = o, p = r) = go[n][o][l] with r = n*L + l, read by
// buffer loads from a descriptor that starts at image n0 (the image of the
// block's first contraction row) and ends at the end of go: rows r >= P lie
// past its end and read 0, so they add nothing whatever the B operand holds,
// and rows o >= O read other images' values, whose results the epilogue
// drops.  The go scale sx * sw[o] is applied to the results instead (it is
// constant along the contraction).  VEC (L % 4 == 0): a quad of rows lies
// in one image, one 16-byte load.  Offsets are 32-bit: the host keeps a
// block's images within 2^31 bytes of go.
template <int B, bool VEC> struct WeightA {
  static constexpr int NQ = B / 32;        // quads per thread (rows m, m+32, ...)
  __amdgpu_buffer_rsrc_t res;
  int O, L;
  int pq, mr, m0;
  int n, l;                 // row p0 + pq: image (from n0) and position
  floatx4 raw[NQ];
  __device__ void init(const float* go, long long go_elems, int t, int mbase, int pb) {
    pq = (t & 7) * 4; mr = t >> 3; m0 = mbase;
    const int n0 = pb / L;
    const long long base = (long long)n0 * O * L;
    const long long bytes = (go_elems - base) * 4;
    res = buffer_rsrc(go + base, (int)(unsigned)(bytes < 0xffffffffLL ? bytes : 0xffffffffLL));
    const int r = pb + pq - n0 * L;
    n = r / L;
    l = r - n * L;
  }
  __device__ void fetch(int, int) {
    const int rowb = 32 * L * 4;           // bytes between a thread's rows o, o + 32
    const unsigned ob = (unsigned)(m0 + mr);
    if constexpr (VEC) {
      const unsigned off = (((unsigned)n * O + ob) * L + l) * 4u;
#pragma unroll
      for (int i = 0; i < NQ; ++i)
        raw[i] = __builtin_bit_cast(floatx4,
                                    __builtin_amdgcn_raw_buffer_load_b128(res, off, i * rowb, 0));
    } else {
      unsigned off[4];
      int en = n, el = l;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        off[e] = (((unsigned)en * O + ob) * L + el) * 4u;
        if (++el == L) { el = 0; ++en; }
      }
#pragma unroll
      for (int i = 0; i < NQ; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          raw[i][e] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(res, off[e], i * rowb, 0));
    }
  }
  template <bool FULL> __device__ void put(char* s, const uint2*) const {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const float v[4] = {raw[i][0], raw[i][1], raw[i][2], raw[i][3]};
      uint2 P[3];
      split4<FULL>(v, P);
      put_parts<B, FULL>(s, mr + 32 * i, pq, P);
    }
  }
  __device__ void advance() {
    l += BK;
    while (l >= L) { l -= L; ++n; }
  }
};

// Backward-weight B: B(p = r, j = k) = tw[index of image tap k at output
// position r] (implicit im2col).  Out-of-image taps use `pad`.  Taps k >= K
// and rows r >= P (whose A values are 0) take the pad entry; the table's
// entries are finite, so those products are 0 or dropped by the epilogue.
template <int B, typename T> struct WeightB {
  static constexpr int NQ = B / 32;
  const T* img; atx_conv_geom g; int K, L, offset, pad;
  int pq, jr;
  int coff[NQ], dh[NQ], dw[NQ];     // per tap: c*H*W, kh*DH - PH, kw*DW - PW
  unsigned kv;                      // bit i: tap i < K
  int n, oh, ow;                    // output position of row p0 + pq
  unsigned raw[NQ][4], in;          // in: element read from the image
  __device__ void init(int t, int n0, int pb) {
    pq = (t & 7) * 4; jr = t >> 3;
    const int KK = g.KH * g.KW;
    kv = 0;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int k = n0 + jr + 32 * i;
      const int kc = k < K ? k : 0;
      const int c = kc / KK, tt = kc - c * KK;
      const int kh = tt / g.KW, kw = tt - kh * g.KW;
      coff[i] = c * g.H * g.W;
      dh[i] = kh * g.DH - g.PH;
      dw[i] = kw * g.DW - g.PW;
      if (k < K) kv |= 1u << i;
    }
    const int r = pb + pq;
    n = r / L;
    const int l = r - n * L;
    oh = l / g.OW;
    ow = l - oh * g.OW;
  }
  __device__ void fetch(int p0, int pe) {
    const int r = p0 + pq;
    in = 0;
    int en = n, eh = oh, ew = ow;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool rv = r + e < pe;
      const long long nb = (long long)en * g.C * g.H * g.W;
      const int ih0 = eh * g.SH, iw0 = ew * g.SW;
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const int ih = ih0 + dh[i], iw = iw0 + dw[i];
        const bool inside = rv && ((kv >> i) & 1u) && (unsigned)ih < (unsigned)g.H &&
                            (unsigned)iw < (unsigned)g.W;
        const T x = img[inside ? nb + coff[i] + ih * g.W + iw : 0];
        if constexpr (sizeof(T) == 4) raw[i][e] = __float_as_uint((float)x);
        else raw[i][e] = (unsigned)(unsigned char)x;
        in |= (inside ? 1u : 0u) << (4 * i + e);
      }
      if (++ew == g.OW) { ew = 0; if (++eh == g.OH) { eh = 0; ++en; } }
    }
  }
  template <bool FULL> __device__ void put(char* s, const uint2* stab) const {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      unsigned idx[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        idx[e] = (in >> (4 * i + e)) & 1u ? img_index<T>(raw[i][e], offset) : (unsigned)pad;
      uint2 P[3];
      lookup4<FULL>(stab, idx, P);
      put_parts<B, FULL>(s, jr + 32 * i, pq, P);
    }
  }
  __device__ void advance() {
    ow += BK;
    while (ow >= g.OW) {
      ow -= g.OW;
      if (++oh == g.OH) { oh = 0; ++n; }
    }
  }
};

// Backward-weight B from the forward's row-offset operand: B(p = r, j = k) =
// tw[xt[slot(k, r)][r] >> 8] (xt as the LUT GEMM reads it: [Kpad][Rpad]
// uint16, slot(k, r) = (k & ~3) | ((k - (r >> 2)) & 3), padding taps and
// rows hold offset 0).  A thread's four rows are one quad and the quad index
// moves by BK / 4 = 8 per k-tile, so each of its taps stays in one slot: one
// 8-byte load per (tap, k-tile) and a bit-field extract per element.  Taps
// k >= K and rows r >= P read padding (finite table entries): their results
// are dropped or multiplied by A's zeros.
template <int B> struct WeightBRows {
  static constexpr int NQ = B / 32;
  const uint16_t* xt; long long Rpad; int K, Kpad;
  int pq, jr;
  const uint16_t* src[NQ];          // slot row of tap i, at the thread's current quad
  uint2 raw[NQ];
  __device__ void init(int t, int n0, int pb) {
    pq = (t & 7) * 4; jr = t >> 3;
    const int r0 = pb + pq;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int k = n0 + jr + 32 * i;
      const int slot = k < Kpad ? ((k & ~3) | ((k - (r0 >> 2)) & 3)) : 0;
      src[i] = xt + (long long)slot * Rpad + r0;
    }
  }
  __device__ void fetch(int, int) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) raw[i] = *(const uint2*)src[i];
  }
  template <bool FULL> __device__ void put(char* s, const uint2* stab) const {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const unsigned w[2] = {raw[i].x, raw[i].y};
      unsigned idx[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) idx[e] = (w[e >> 1] >> (16 * (e & 1) + 8)) & 255u;
      uint2 P[3];
      lookup4<FULL>(stab, idx, P);
      put_parts<B, FULL>(s, jr + 32 * i, pq, P);
    }
  }
  __device__ void advance() {
#pragma unroll
    for (int i = 0; i < NQ; ++i) src[i] += BK;
  }
};

// ---------------------------------------- backward-data loaders (bf16 planes)
// Backward-data A from prepared planes [3][Kp][Opad] (the h, m, l parts of
// tx[wq[o][k]], zero for k >= K and o >= O; Kp, Opad multiples of 128 and
// 32): A(m = k, p = o).  Row m of a k-tile is 64 contiguous bytes per
// plane; a thread copies 16-byte units (three planes, or only the h plane
// when the table is bf16 exactly).  Buffer loads: rows past the planes read
// 0.  DGRAD: rows m = input channel c of the implicit GEMM, whose k-tile
// p0 holds tap t = p0 / O (O % 32 == 0): source row c*KK + t, columns from
// p0 - t*O.
template <int B, bool DGRAD> struct PlaneA {
  static constexpr int NU = 3 * B * 4 / GT;   // 16-byte units per thread, three planes
  const uint16_t* planes; int pbytes;        // the planes and their size
  __amdgpu_buffer_rsrc_t res;
  int Kp, Opad, KK, O, m0, t;
  bool full;
  u32x4 raw[NU];
  __device__ void init(int tid, int mbase) {
    t = tid; m0 = mbase;
    res = buffer_rsrc(planes, pbytes);
  }
  __device__ void fetch(int p0, int) {
    int tap = 0, o0 = p0;
    if constexpr (DGRAD) { tap = p0 / O; o0 = p0 - tap * O; }
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      if (j >= NU / 3 && !full) break;
      const int u = t + GT * j;
      const int q = u / (4 * B), row = (u >> 2) % B, unit = u & 3;
      const int src = DGRAD ? (m0 + row) * KK + tap : m0 + row;
      const unsigned off = (((unsigned)q * Kp + src) * Opad + o0 + 8 * unit) * 2u;
      raw[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(res, off, 0, 0));
    }
  }
  template <bool FULL> __device__ void put(char* s, const uint2*) const {
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      if (j >= NU / 3 && !FULL) break;
      const int u = t + GT * j;
      const int q = u / (4 * B), row = (u >> 2) % B, unit = u & 3;
      *(u32x4*)(s + q * Planes<B>::PLANE + Planes<B>::at(row, 8 * unit)) = raw[j];
    }
  }
  __device__ void advance() {}
};

// Backward-data B: B(p = o, col = c) = go[n][o][l] * fp32(sx * sw[o]) with
// c = n*L + l (the product of scales rounded first, the order of the layer's
// `y * (scale_x * scale_w)`).  A thread holds four columns x four
// consecutive o (o-quad oq = t & 7, column quad cq = t >> 3) and stores each
// column's four contraction elements as 8-byte plane groups.  Buffer loads
// from a descriptor starting at the block's first image: columns past N*L
// read 0 (offset 2^31, past the descriptor), o >= O reads the next image's
// values or 0 (the A planes are 0 there).  VEC (L % 4 == 0): a column quad
// lies in one image, one 16-byte load per o.
template <int B, bool VEC, bool SCALED> struct GoCols {
  static_assert(B == 128, "GoCols covers 128 columns with 256 threads");
  __amdgpu_buffer_rsrc_t res;
  int O, L;
  const float* sx; const float* sw;
  int oq, cq;
  unsigned off[4];          // byte offset of column 4cq + e at o = 0 (VEC: off[0] only)
  floatx4 raw[4];           // raw[i][e]: o = p0 + 4oq + i, column 4cq + e
  float sc[4];
  __device__ void init(const float* go, long long go_elems, int tid, int n0, int NL) {
    oq = tid & 7; cq = tid >> 3;
    const int nb = n0 / L;
    const long long base = (long long)nb * O * L;
    const long long bytes = (go_elems - base) * 4;
    res = buffer_rsrc(go + base, (int)(bytes < 0x7fffffffLL ? bytes : 0x7fffffffLL));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = n0 + 4 * cq + e;
      const int n = c / L;
      off[e] = c < NL ? (unsigned)(((long long)(n - nb) * O * L + (c - n * L)) * 4) : 0x80000000u;
    }
  }
  __device__ void fetch(int p0, int) {
    const int ob = p0 + 4 * oq;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const unsigned ol = (unsigned)(ob + i) * L * 4u;
      if constexpr (SCALED) sc[i] = sx[0] * sw[ob + i < O ? ob + i : 0];
      if constexpr (VEC) {
        raw[i] = __builtin_bit_cast(floatx4,
                                    __builtin_amdgcn_raw_buffer_load_b128(res, off[0] + ol, 0, 0));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          raw[i][e] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(res, off[e] + ol, 0, 0));
      }
    }
    // The last, partial k-tile reads rows o >= O (the next image's), whose
    // weight planes are zero: zero them here too, so that a non-finite go
    // there cannot add 0 * inf = NaN.  p0 is the tile start (wave-uniform).
    if (p0 + 32 > O) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (ob + i >= O) raw[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  template <bool FULL> __device__ void put(char* s, const uint2*) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = SCALED ? raw[i][e] * sc[i] : raw[i][e];
      uint2 P[3];
      split4<FULL>(v, P);
      put_parts<B, FULL>(s, 4 * cq + e, 4 * oq, P);
    }
  }
  __device__ void advance() {}
};

// Implicit backward-data B: B(p = t*O + o, col = (n, h, w)) =
// go'[n, o, h + PH - i*DH, w + PW - j*DW] (tap t = i*KW + j, uniform over a
// k-tile since O % 32 == 0; zero outside go), with GoCols' thread layout
// and scaling.  Elements outside the image use offset 2^31 (read 0).
template <int B, bool SCALED> struct ShiftCols {
  static_assert(B == 128, "ShiftCols covers 128 columns with 256 threads");
  __amdgpu_buffer_rsrc_t res;
  atx_conv_geom g; int O;
  const float* sx; const float* sw;
  int oq, cq;
  int nb[4], hh[4], ww[4];  // image offset (elements, from the descriptor base; -1: none), pixel
  floatx4 raw[4];
  float sc[4];
  __device__ void init(const float* go, long long go_elems, int tid, int n0, int NHW) {
    oq = tid & 7; cq = tid >> 3;
    const int HW = g.H * g.W;
    const long long OHW = (long long)g.OH * g.OW;
    const int nbase = n0 / HW;
    const long long base = (long long)nbase * O * OHW;
    const long long bytes = (go_elems - base) * 4;
    res = buffer_rsrc(go + base, (int)(bytes < 0x7fffffffLL ? bytes : 0x7fffffffLL));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = n0 + 4 * cq + e;
      if (c < NHW) {
        const int n = c / HW, hw = c - n * HW;
        hh[e] = hw / g.W;
        ww[e] = hw - hh[e] * g.W;
        nb[e] = (int)((n - nbase) * O * OHW);
      } else {
        nb[e] = -1; hh[e] = ww[e] = 0;
      }
    }
  }
  __device__ void fetch(int p0, int) {
    const int tap = p0 / O, o0 = p0 - tap * O;
    const int ki = tap / g.KW, kj = tap - ki * g.KW;
    const int dh0 = g.PH - ki * g.DH, dw0 = g.PW - kj * g.DW;
    const int OHW = g.OH * g.OW;
    unsigned off[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ih = hh[e] + dh0, iw = ww[e] + dw0;
      const bool v = nb[e] >= 0 && (unsigned)ih < (unsigned)g.OH && (unsigned)iw < (unsigned)g.OW;
      off[e] = v ? (unsigned)(nb[e] + ih * g.OW + iw) * 4u : 0x80000000u;
    }
    const int ob = o0 + 4 * oq;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const unsigned ol = (unsigned)(ob + i) * OHW * 4u;
      if constexpr (SCALED) sc[i] = sx[0] * sw[ob + i];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        raw[i][e] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(res, off[e] + ol, 0, 0));
    }
  }
  template <bool FULL> __device__ void put(char* s, const uint2*) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = SCALED ? raw[i][e] * sc[i] : raw[i][e];
      uint2 P[3];
      split4<FULL>(v, P);
      put_parts<B, FULL>(s, 4 * cq + e, 4 * oq, P);
    }
  }
  __device__ void advance() {}
};

// ------------------------------------------------------------------ epilogues
// out[n][k][l] of the backward-data GEMM (rows m = k, columns c = n*L + l).
// With `mask`, the fake-quant STE is applied on the way out:
// v = (mask ? v : 0) / max(scale, 1e-12) (the 1x1 stride-1 conv, whose
// columns are the image gradient itself).
struct DataOut {
  float* col; int K, L, NL;
  const uint8_t* mask; const float* scale;
  long long split_stride;   // elements per partial slice (blockIdx.z = slice)
};
// ws[s][o][k] of the backward-weight GEMM, times the go scale sx * sw[o]
// when sw is given.
struct WeightOut {
  float* ws; int O, K; long long sst;
  const float* sx; const float* sw;
  __device__ void store(int m, int c, float v, int s) const {
    if (m < O && c < K) {
      if (sw) v *= sx[0] * sw[m];
      ws[(long long)s * sst + (long long)m * K + c] = v;
    }
  }
};

// ----------------------------------------------------------------- main kernel
// TR: the MFMA takes the B fragment as its first operand, so the 16x16
// result block is stored transposed (lane holds columns 4*(lane >> 4) + r of
// row lane & 15); the products and their order are the same.
template <int BM, int BN, class LA, class LB, bool TR = false>
__device__ __forceinline__ void mma_tile(const float* As, const float* Bs,
                                         floatx4 (&acc)[BM / 32][BN / 32]) {
  constexpr int TM = BM / 32, TN = BN / 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 15, lk = lane >> 4;
#pragma unroll
  for (int kk = 0; kk < BK; kk += 4) {
    float a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = As[LA::Lay::at(wm * (BM / 2) + i * 16 + li, kk + lk)];
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = Bs[LB::Lay::at(wn * (BN / 2) + j * 16 + li, kk + lk)];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = TR ? __builtin_amdgcn_mfma_f32_16x16x4f32(b[j], a[i], acc[i][j], 0, 0, 0)
                       : __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// acc = sum over the contraction range [pb, pe) of A tile x B tile.
// Double-buffered: the global loads of k-tile i+1 are in flight while tile i
// is multiplied; one barrier per k-tile.
template <int BM, int BN, bool TR = false, class LA, class LB>
__device__ __forceinline__ void gemm_tiles(LA& la, LB& lb, const float* tab, int pb, int pe,
                                           floatx4 (&acc)[BM / 32][BN / 32], float* As0,
                                           float* As1, float* Bs0, float* Bs1) {
#pragma unroll
  for (int i = 0; i < BM / 32; ++i)
#pragma unroll
    for (int j = 0; j < BN / 32; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  if (pb >= pe) return;

  la.fetch(pb, pe);
  lb.fetch(pb, pe);
  la.stash(As0, tab);
  lb.stash(Bs0, tab);
  __syncthreads();
  float *Ac = As0, *An = As1, *Bc = Bs0, *Bn = Bs1;
  for (int p0 = pb; p0 + BK < pe; p0 += BK) {
    la.advance(); lb.advance();
    la.fetch(p0 + BK, pe);
    lb.fetch(p0 + BK, pe);
    // Keep the next tile's loads ahead of the MFMAs and their consumers
    // behind them: the scheduler would otherwise sink the loads, or hoist
    // the stash's use of them, and expose the load latency.
    __builtin_amdgcn_sched_barrier(0);
    mma_tile<BM, BN, LA, LB, TR>(Ac, Bc, acc);
    __builtin_amdgcn_sched_barrier(0);
    la.stash(An, tab);
    lb.stash(Bn, tab);
    __syncthreads();
    float* x = Ac; Ac = An; An = x;
    x = Bc; Bc = Bn; Bn = x;
  }
  mma_tile<BM, BN, LA, LB, TR>(Ac, Bc, acc);
}

// acc += A tile x B tile from split-bf16 planes (one 32-deep MFMA step).
// Lane (i = lane & 15, g = lane >> 4) reads 16 bytes (contraction elements
// 8g..8g+7) of row i of each 16-row block; the result blocks have the fp32
// path's layout (lane holds rows 4g + r of column i).  The part products are
// added smallest first.
// TR: the B fragment is the MFMA's first operand, so each 16x16 result block
// comes out transposed (lane holds columns 4*(lane >> 4) + r of row
// lane & 15), the layout of the data epilogue's vector path.
template <int BM, int BN, int PR, bool TR = false>
__device__ __forceinline__ void mma_planes(const char* As, const char* Bs,
                                           floatx4 (&acc)[BM / 32][BN / 32]) {
  constexpr int TM = BM / 32, TN = BN / 32;
  constexpr int NA = PR == A_EXACT ? 1 : 3;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 15, k8 = 8 * (lane >> 4);
  // A parts stay in registers; the B parts are read one at a time, each
  // taking its products with the A parts of total order <= 2 (smallest
  // first: B part q with A parts 2 - q .. 0).
  u32x4 a[NA][TM];
#pragma unroll
  for (int q = 0; q < NA; ++q)
#pragma unroll
    for (int i = 0; i < TM; ++i)
      a[q][i] = *(const u32x4*)(As + q * Planes<BM>::PLANE +
                                Planes<BM>::at(wm * (BM / 2) + i * 16 + li, k8));
  constexpr int NB = PR == B_EXACT ? 1 : 3;
#pragma unroll
  for (int q = 0; q < NB; ++q) {
    u32x4 b[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j)
      b[j] = *(const u32x4*)(Bs + q * Planes<BN>::PLANE +
                             Planes<BN>::at(wn * (BN / 2) + j * 16 + li, k8));
#pragma unroll
    for (int qa = (PR == A_EXACT ? 0 : 2 - q); qa >= 0; --qa)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = TR ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                               __builtin_bit_cast(bf16x8, b[j]), __builtin_bit_cast(bf16x8, a[qa][i]),
                               acc[i][j], 0, 0, 0)
                         : __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                               __builtin_bit_cast(bf16x8, a[qa][i]), __builtin_bit_cast(bf16x8, b[j]),
                               acc[i][j], 0, 0, 0);
  }
}

// acc = sum over the contraction range [pb, pe) on split-bf16 planes.  One
// LDS tile per operand: the loaders' global loads of k-tile i+1 are in
// flight while tile i is multiplied, then stored as planes after a barrier
// (two barriers per k-tile; the kernels run two blocks per CU, so one
// block's MFMAs cover the other's stores).
template <int BM, int BN, int PR, bool TR = false, class LA, class LB>
__device__ __forceinline__ void gemm_planes(LA& la, LB& lb, const uint2* stab, int pb, int pe,
                                            floatx4 (&acc)[BM / 32][BN / 32], char* As,
                                            char* Bs) {
#pragma unroll
  for (int i = 0; i < BM / 32; ++i)
#pragma unroll
    for (int j = 0; j < BN / 32; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  if (pb >= pe) return;
  la.fetch(pb, pe);
  lb.fetch(pb, pe);
  for (int p0 = pb;; p0 += BK) {
    la.template put<PR != A_EXACT>(As, stab);
    lb.template put<PR != B_EXACT>(Bs, stab);
    __syncthreads();
    const bool more = p0 + BK < pe;
    if (more) {
      la.advance(); lb.advance();
      la.fetch(p0 + BK, pe);
      lb.fetch(p0 + BK, pe);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma_planes<BM, BN, PR, TR>(As, Bs, acc);
    if (!more) break;
    __syncthreads();
  }
}

// Data-GEMM epilogue: out[n][m][l] for column c = n*L + l (rows m), with the
// optional per-tensor fake-quant STE (mask ? v : 0) / max(scale, 1e-12).
// VEC (L % 4 == 0, out 16-byte and mask 4-byte aligned): the tiles are
// multiplied with TR (transposed 16x16 blocks), so a lane holds the four
// consecutive columns c0..c0+3 of one row m; the quad lies in one image and
// is wholly inside N*L or wholly outside, so it is one 16-byte store and one
// 4-byte mask load.  Otherwise the blocks are untransposed and every element
// is stored on its own.
template <int BM, int BN, bool VEC>
__device__ __forceinline__ void data_epilogue(const DataOut& ep,
                                              const floatx4 (&acc)[BM / 32][BN / 32], int m0,
                                              int n0) {
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  constexpr int TM = BM / 32;
  const float sdiv = ep.mask ? fmaxf(ep.scale[0], 1e-12f) : 1.0f;
  if constexpr (VEC) {
#pragma unroll
  for (int j = 0; j < BN / 32; ++j) {
    const int c0 = n0 + wn * (BN / 2) + j * 16 + 4 * (lane >> 4);
    {
      const bool cv = c0 < ep.NL;
      const int cc = cv ? c0 : 0;
      const int n = cc / ep.L;
      const long long off = (long long)n * ep.K * ep.L + (cc - n * ep.L);
      if (ep.mask) {
        unsigned mk[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = m0 + wm * (BM / 2) + i * 16 + (lane & 15);
          mk[i] = *(const unsigned*)(ep.mask + (cv && m < ep.K ? off + (long long)m * ep.L : 0));
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = m0 + wm * (BM / 2) + i * 16 + (lane & 15);
          floatx4 v;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[r] = ((mk[i] >> (8 * r)) & 255u ? acc[i][j][r] : 0.0f) / sdiv;
          if (cv && m < ep.K) *(floatx4*)(ep.col + off + (long long)m * ep.L) = v;
        }
      } else {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = m0 + wm * (BM / 2) + i * 16 + (lane & 15);
          if (cv && m < ep.K) *(floatx4*)(ep.col + off + (long long)m * ep.L) = acc[i][j];
        }
      }
    }
  }
  } else {
    // untransposed blocks (lane holds rows 4*(lane >> 4) + r of column
    // lane & 15): per element, 16 consecutive columns per store
#pragma unroll
    for (int j = 0; j < BN / 32; ++j) {
      const int c = n0 + wn * (BN / 2) + j * 16 + (lane & 15);
      const bool cv = c < ep.NL;
      const int cc = cv ? c : 0;
      const int n = cc / ep.L;
      const long long off = (long long)n * ep.K * ep.L + (cc - n * ep.L);
      if (ep.mask) {
        unsigned char mk[TM][4];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + r;
            mk[i][r] = ep.mask[cv && m < ep.K ? off + (long long)m * ep.L : 0];
          }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + r;
            if (cv && m < ep.K)
              ep.col[off + (long long)m * ep.L] = (mk[i][r] ? acc[i][j][r] : 0.0f) / sdiv;
          }
      } else {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + r;
            if (cv && m < ep.K) ep.col[off + (long long)m * ep.L] = acc[i][j][r];
          }
      }
    }
  }
}


// VB: go quads (L % 4 == 0) are 16-byte loads and the output quads 16-byte
// stores (data_epilogue VEC).
template <int BM, int BN, bool VA, bool VB, bool SC>
__global__ void __launch_bounds__(GT, 2)
data_gemm_kernel(DataA<BM, VA> la, DataB<BN, VB, SC> lb, DataOut ep,
                 const float* __restrict__ tx, int O, int o_chunk) {
  __shared__ float tab[256];
  __shared__ __align__(16) float As[2][KMajor<BM>::SIZE];
  __shared__ __align__(16) float Bs[2][KMajor<BN>::SIZE];
  const int t = threadIdx.x;
  tab[t] = tx[t];
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  la.init(t, m0);
  lb.init(t, n0);
  __syncthreads();
  // contraction slice of this block (grid.z splits O; each slice writes its
  // own partial output, summed afterwards in a fixed order)
  const int ob = blockIdx.z * o_chunk, oe = min(O, ob + o_chunk);
  ep.col += (long long)blockIdx.z * ep.split_stride;
  floatx4 acc[BM / 32][BN / 32];
  gemm_tiles<BM, BN, VB>(la, lb, tab, ob, oe, acc, As[0], As[1], Bs[0], Bs[1]);
  data_epilogue<BM, BN, VB>(ep, acc, m0, n0);
}

// Implicit backward-data kernel: the data GEMM's epilogue (direct image
// output with the optional fused STE) over DgradA x DgradB.
template <int BM, int BN, bool SC, bool VO>
__global__ void __launch_bounds__(GT, 2)
dgrad_gemm_kernel(DgradA<BM> la, DgradB<BN, SC> lb, DataOut ep, const float* __restrict__ tx,
                  int P) {
  __shared__ float tab[256];
  __shared__ __align__(16) float As[2][KMajor<BM>::SIZE];
  __shared__ __align__(16) float Bs[2][KMajor<BN>::SIZE];
  const int t = threadIdx.x;
  tab[t] = tx[t];
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  la.init(t, m0);
  lb.init(t, n0);
  __syncthreads();
  floatx4 acc[BM / 32][BN / 32];
  gemm_tiles<BM, BN, VO>(la, lb, tab, 0, P, acc, As[0], As[1], Bs[0], Bs[1]);
  data_epilogue<BM, BN, VO>(ep, acc, m0, n0);
}

// planes[q][k][o] (q = h, m, l part of tx[wq[o*K + k]]; zero for k >= K or
// o >= O) over Kp x Opad, the A operand of the plane data GEMMs.  A thread
// writes eight consecutive o of one k per plane (16 bytes).
__global__ void __launch_bounds__(GT)
weight_planes_kernel(const uint8_t* __restrict__ wq, const float* __restrict__ tx, int O, int K,
                     int Kp, int Opad, uint16_t* __restrict__ planes) {
  __shared__ uint2 stab[257];
  split_table(stab, tx, threadIdx.x);
  const long long idx = (long long)blockIdx.x * GT + threadIdx.x;
  const int per_row = Opad / 8;
  if (idx >= (long long)Kp * per_row) return;
  const int k = (int)(idx / per_row), o8 = (int)(idx - (long long)k * per_row) * 8;
  uint2 P[2][3];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    unsigned ix[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int o = o8 + 4 * h + e;
      ix[e] = k < K && o < O ? wq[(long long)o * K + k] : 256u;
    }
    lookup4<true>(stab, ix, P[h]);
  }
  const long long plane = (long long)Kp * Opad;
#pragma unroll
  for (int q = 0; q < 3; ++q)
    *(uint4*)(planes + q * plane + (long long)k * Opad + o8) =
        make_uint4(P[0][q].x, P[0][q].y, P[1][q].x, P[1][q].y);
}

// Backward-data GEMM on split-bf16 planes: A from weight_planes_kernel's
// planes (three parts, or one when the table is bf16 exactly), B = go (six
// part products, or three).  VB (L % 4 == 0): 16-byte go loads and the
// transposed epilogue.  Two blocks per CU.
template <int BM, bool VB, bool SC>
__global__ void __launch_bounds__(GT, 2)
data_planes_kernel(PlaneA<BM, false> la, GoCols<128, VB, SC> lb, DataOut ep,
                   const float* __restrict__ go, long long go_elems,
                   const float* __restrict__ tx, int O, int o_chunk) {
  __shared__ __align__(16) char As[Planes<BM>::SIZE];
  __shared__ __align__(16) char Bs[Planes<128>::SIZE];
  const int t = threadIdx.x;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * 128;
  la.init(t, m0);
  lb.init(go, go_elems, t, n0, ep.NL);
  const bool exact = table_exact(tx, t);
  la.full = !exact;
  const int ob = blockIdx.z * o_chunk, oe = min(O, ob + o_chunk);
  ep.col += (long long)blockIdx.z * ep.split_stride;
  floatx4 acc[BM / 32][4];
  if (exact) gemm_planes<BM, 128, A_EXACT, VB>(la, lb, nullptr, ob, oe, acc, As, Bs);
  else gemm_planes<BM, 128, PROD6, VB>(la, lb, nullptr, ob, oe, acc, As, Bs);
  data_epilogue<BM, 128, VB>(ep, acc, m0, n0);
}

// Implicit backward-data GEMM on split-bf16 planes (A rows c*KK + t of the
// prepared planes, B = shifted go).  VO: 16-byte output stores.
template <int BM, bool SC, bool VO>
__global__ void __launch_bounds__(GT, 2)
dgrad_planes_kernel(PlaneA<BM, true> la, ShiftCols<128, SC> lb, DataOut ep,
                    const float* __restrict__ go, long long go_elems,
                    const float* __restrict__ tx, int P) {
  __shared__ __align__(16) char As[Planes<BM>::SIZE];
  __shared__ __align__(16) char Bs[Planes<128>::SIZE];
  const int t = threadIdx.x;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * 128;
  la.init(t, m0);
  lb.init(go, go_elems, t, n0, ep.NL);
  const bool exact = table_exact(tx, t);
  la.full = !exact;
  floatx4 acc[BM / 32][4];
  if (exact) gemm_planes<BM, 128, A_EXACT, VO>(la, lb, nullptr, 0, P, acc, As, Bs);
  else gemm_planes<BM, 128, PROD6, VO>(la, lb, nullptr, 0, P, acc, As, Bs);
  data_epilogue<BM, 128, VO>(ep, acc, m0, n0);
}

template <class LB> __device__ __forceinline__ void set_pad(LB&, const float*) {}
template <int B, typename T>
__device__ __forceinline__ void set_pad(WeightB<B, T>& lb, const float* pad_dev) {
  if (pad_dev) lb.pad = (int)quant_index(pad_dev[0], 0);
}

// Backward-weight GEMM on split-bf16 planes: A = go (six part products),
// B = the table (three when every table entry is bf16 exactly).
template <int BM, int BN, bool VA, class LB>
__global__ void __launch_bounds__(GT, 2)
weight_gemm_kernel(WeightA<BM, VA> la, LB lb, WeightOut ep, const float* __restrict__ go,
                   long long go_elems, const float* __restrict__ tw,
                   const float* __restrict__ pad_dev, int P, int p_chunk) {
  __shared__ uint2 stab[257];
  __shared__ __align__(16) char As[Planes<BM>::SIZE];
  __shared__ __align__(16) char Bs[Planes<BN>::SIZE];
  const int t = threadIdx.x;
  set_pad(lb, pad_dev);
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int s = blockIdx.z;
  const int pb = s * p_chunk, pe = min(P, pb + p_chunk);
  la.init(go, go_elems, t, m0, pb);
  lb.init(t, n0, pb);
  const bool exact = split_table(stab, tw, t);
  floatx4 acc[BM / 32][BN / 32];
  if (exact) gemm_planes<BM, BN, B_EXACT>(la, lb, stab, pb, pe, acc, As, Bs);
  else gemm_planes<BM, BN, PROD6>(la, lb, stab, pb, pe, acc, As, Bs);
  const int lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < BM / 32; ++i)
#pragma unroll
    for (int j = 0; j < BN / 32; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ep.store(m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + r,
                 n0 + wn * (BN / 2) + j * 16 + (lane & 15), acc[i][j][r], s);
}

// gw[i] = sum_s ws[s][i]; optional per-channel term (the uint8 layer's weight
// zero point): gw -= (zsum[o] * (zsx * scale[o])) * zzx, each product and the
// difference rounded on its own; optional fused per-channel fake-quant
// backward: gw = mask ? gw / max(scale[o], 1e-12) : 0 with o = i / K.  A block
// sums 256 / G consecutive elements over G groups of slices (group g takes
// slices g, g + G, ...), then adds the G partials in group order:
// deterministic.
template <bool VEC>
__global__ void __launch_bounds__(256)
split_sum_kernel(const float* __restrict__ ws, int S, long long numel, int K, int G,
                 const uint8_t* __restrict__ mask, const float* __restrict__ scale,
                 float* __restrict__ out, const float* __restrict__ zsum,
                 const float* __restrict__ zsx, const float* __restrict__ zzx) {
  // VEC: each item is four consecutive elements (16-byte loads and stores;
  // numel % 4 == 0); every element keeps the same summation order.
  constexpr int W = VEC ? 4 : 1;
  typedef float floatw __attribute__((ext_vector_type(W)));
  __shared__ floatw part[256];
  const int t = threadIdx.x;
  const int epb = 256 / G;
  const int e = t % epb, grp = t / epb;
  const long long i = ((long long)blockIdx.x * epb + e) * W;   // first element
  floatw a = 0.0f;
  if (i < numel)
    for (int s = grp; s < S; s += G) a += *(const floatw*)(ws + (long long)s * numel + i);
  part[t] = a;
  __syncthreads();
  if (grp == 0 && i < numel) {
    for (int g = 1; g < G; ++g) a += part[g * epb + e];
    if (mask || zsum) {
      long long o = i / K, r = i - o * K;
#pragma unroll
      for (int j = 0; j < W; ++j) {
        float v = a[j];
        if (zsum) {
#pragma clang fp contract(off)
          v = v - (zsum[o] * (zsx[0] * scale[o])) * zzx[0];
        }
        if (mask) v = (mask[i + j] ? v : 0.0f) / fmaxf(scale[o], 1e-12f);
        a[j] = v;
        if (++r == K) { r = 0; ++o; }
      }
    }
    *(floatw*)(out + i) = a;
  }
}

// Launch of split_sum_kernel: enough groups that the grid has >= 1024 blocks.
int launch_split_sum(const float* ws, int S, long long numel, int K,
                            const uint8_t* mask, const float* scale, float* out,
                            hipStream_t stream, const float* zsum, const float* zsx,
                            const float* zzx) {
  const bool vec = numel % 4 == 0 && ((uintptr_t)ws & 15) == 0 && ((uintptr_t)out & 15) == 0;
  const long long items = vec ? numel / 4 : numel;
  int G = 1;
  while (G < 64 && G < S && cdiv(items, 256 / G) < 1024) G *= 2;
  const long long blocks = cdiv(items, 256 / G);
  ATX_REQUIRE(blocks <= 0x7fffffffLL, "split_sum: too many elements");
  if (vec)
    hipLaunchKernelGGL(split_sum_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       ws, S, numel, K, G, mask, scale, out, zsum, zsx, zzx);
  else
    hipLaunchKernelGGL(split_sum_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       ws, S, numel, K, G, mask, scale, out, zsum, zsx, zzx);
  return check_launch("split_sum_kernel");
}

inline int tile_of(int extent) { return extent <= 64 ? 64 : 128; }

// Split of the weight-gradient contraction, every split at least four
// k-tiles deep.  Cost in k-tiles: rounds of 512 blocks (two per CU) x
// (k-tiles per block + 4 for the block's prologue and epilogue) + 2 + S x
// O*K / 1.5e6 for writing and summing the S partial slices.  Any S, not just
// powers of two: one round with many k-tiles per block beats several rounds
// with few (each block's pipeline start and epilogue are paid per round).
static int weight_splits(int O, int K, long long P) {
  const long long tiles = cdiv(O, tile_of(O)) * cdiv(K, tile_of(K));
  const long long kt = cdiv(P, BK);                 // k-tiles of the contraction
  const long long smax = std::max<long long>(1, std::min<long long>(P / (4 * BK), 4096));
  double best = 0.0;
  long long pick = 1;
  for (long long s = 1; s <= smax; ++s) {
    const long long kc = cdiv(kt, s), sr = cdiv(kt, kc);
    // each split's rows of go within 1 GiB (32-bit buffer offsets)
    if ((double)kc * BK * O * 4.0 > (double)(1LL << 30) && s < smax) continue;
    const double cost = (double)cdiv(tiles * sr, 512) * (kc + 4) +
                        (sr > 1 ? 2.0 + (double)sr * O * K / 1.5e6 : 0.0);
    if (best == 0.0 || cost < best) { best = cost; pick = sr; }
  }
  return (int)pick;
}

struct DataArgs {
  const float* go; const uint8_t* wq; const float* tx; int N, O, K, L;
  const float* sx; const float* sw;          // optional go scale sx * sw[o]
  float* out; const uint8_t* mask; const float* scale;
  int splits, o_chunk;                       // contraction split (1 = none)
  float* partials;                           // [splits][N*K*L] when splits > 1
  uint16_t* planes;                          // bf16 weight planes (null: fp32 kernels)
};

// Bytes of the bf16 weight planes [3][Kp][Opad] (Kp = K rounded up to 128,
// Opad = O rounded up to 32; a multiple of 256 bytes).
static long long weight_planes_bytes(int K, int O) {
  return 3LL * cdiv(K, 128) * 128 * cdiv(O, BK) * BK * 2;
}

// go spans of at most 2^31 bytes per block (32-bit buffer offsets): the
// images a block's 128 columns touch, two partial images included.
static bool planes_fit(long long cols_per_image, int O, long long out_per_image) {
  return (cdiv(128, cols_per_image) + 2) * (long long)O * out_per_image * 4 < (1LL << 31);
}

static int launch_weight_planes(const uint8_t* wq, const float* tx, int O, int K,
                                uint16_t* planes, hipStream_t stream) {
  const int Kp = (int)(cdiv(K, 128) * 128), Opad = (int)(cdiv(O, BK) * BK);
  const long long items = (long long)Kp * (Opad / 8);
  hipLaunchKernelGGL(weight_planes_kernel, dim3((unsigned)cdiv(items, GT)), dim3(GT), 0, stream,
                     wq, tx, O, K, Kp, Opad, planes);
  return check_launch("weight_planes_kernel");
}

// Split of the backward-data contraction over O into deterministic partial
// slices, each at least four k-tiles deep.  Cost in k-tiles, as for the
// weight gradient: rounds of 512 blocks x (k-tiles per block + 4) + 2 + S x
// N*K*L / 1.5e6 for writing and summing the partials (the output is the
// col buffer or the image gradient, so a split pays only when the tiles
// leave most of a round idle).
static int data_splits(int N, int O, int K, int L) {
  const long long blocks = cdiv((long long)N * L, 128) * cdiv(K, tile_of(K));
  const long long numel = (long long)N * K * L;
  if (numel > 0x7fffffffLL) return 1;
  const long long kt = cdiv(O, BK);
  const long long smax = std::max<long long>(1, std::min<long long>(kt / 4, 64));
  double best = 0.0;
  long long pick = 1;
  for (long long s = 1; s <= smax; ++s) {
    const long long kc = cdiv(kt, s), sr = cdiv(kt, kc);
    const double cost = (double)cdiv(blocks * sr, 512) * (kc + 4) +
                        (sr > 1 ? 2.0 + (double)sr * numel / 1.5e6 : 0.0);
    if (s == 1 || cost < best) { best = cost; pick = sr; }
  }
  return (int)pick;
}

template <int BM, bool VA, bool VB, bool SC>
static void launch_data(const DataArgs& a, hipStream_t stream) {
  constexpr int BN = 128;
  const int NL = a.N * a.L;
  DataA<BM, VA> la{};
  la.wq = a.wq; la.K = a.K;
  DataB<BN, VB, SC> lb{};
  lb.go = a.go; lb.O = a.O; lb.L = a.L; lb.NL = NL; lb.sx = a.sx; lb.sw = a.sw;
  const bool split = a.splits > 1;
  DataOut ep{split ? a.partials : a.out, a.K, a.L, NL, split ? nullptr : a.mask,
             split ? nullptr : a.scale, (long long)NL * a.K};
  dim3 grid((unsigned)cdiv(NL, BN), (unsigned)cdiv(a.K, BM), (unsigned)a.splits);
  hipLaunchKernelGGL((data_gemm_kernel<BM, BN, VA, VB, SC>), grid, dim3(GT), 0, stream, la, lb,
                     ep, a.tx, a.O, a.o_chunk);
}

template <int BM, bool VB, bool SC>
static void launch_data_planes(const DataArgs& a, hipStream_t stream) {
  const int NL = a.N * a.L;
  PlaneA<BM, false> la{};
  la.planes = a.planes; la.pbytes = (int)weight_planes_bytes(a.K, a.O);
  la.Kp = (int)(cdiv(a.K, 128) * 128); la.Opad = (int)(cdiv(a.O, BK) * BK);
  GoCols<128, VB, SC> lb{};
  lb.O = a.O; lb.L = a.L; lb.sx = a.sx; lb.sw = a.sw;
  const bool split = a.splits > 1;
  DataOut ep{split ? a.partials : a.out, a.K, a.L, NL, split ? nullptr : a.mask,
             split ? nullptr : a.scale, (long long)NL * a.K};
  dim3 grid((unsigned)cdiv(NL, 128), (unsigned)cdiv(a.K, BM), (unsigned)a.splits);
  hipLaunchKernelGGL((data_planes_kernel<BM, VB, SC>), grid, dim3(GT), 0, stream, la, lb, ep,
                     a.go, (long long)a.N * a.O * a.L, a.tx, a.O, a.o_chunk);
}

template <int BM, bool SC>
static void dispatch_data_vec(const DataArgs& a, hipStream_t stream) {
  const bool va = a.K % 4 == 0 && (uintptr_t)a.wq % 4 == 0;
  const float* out = a.splits > 1 ? a.partials : a.out;
  const bool vb = a.L % 4 == 0 && (uintptr_t)a.go % 16 == 0 && (uintptr_t)out % 16 == 0 &&
                  (a.splits > 1 || (uintptr_t)a.mask % 4 == 0);
  if (a.planes) {
    if (vb) launch_data_planes<BM, true, SC>(a, stream);
    else launch_data_planes<BM, false, SC>(a, stream);
    return;
  }
  if (va && vb) launch_data<BM, true, true, SC>(a, stream);
  else if (va) launch_data<BM, true, false, SC>(a, stream);
  else if (vb) launch_data<BM, false, true, SC>(a, stream);
  else launch_data<BM, false, false, SC>(a, stream);
}

// Runs the backward-data GEMM into a.out; with a.splits > 1 the partial
// slices go to a.partials and are summed into a.out (with the optional
// per-tensor STE mask) by split_sum_kernel.
static int run_data_gemm(DataArgs a, hipStream_t stream) {
  if (a.splits < 1) a.splits = 1;
  a.o_chunk = (int)(cdiv(cdiv(a.O, a.splits), BK) * BK);
  a.splits = (int)cdiv(a.O, a.o_chunk);
  if (a.planes && !planes_fit(a.L, a.O, a.L)) a.planes = nullptr;
  if (a.planes) {
    const int rc = launch_weight_planes(a.wq, a.tx, a.O, a.K, a.planes, stream);
    if (rc) return rc;
  }
  const bool sc = a.sw != nullptr;
  if (tile_of(a.K) == 64) {
    if (sc) dispatch_data_vec<64, true>(a, stream); else dispatch_data_vec<64, false>(a, stream);
  } else {
    if (sc) dispatch_data_vec<128, true>(a, stream); else dispatch_data_vec<128, false>(a, stream);
  }
  int rc = check_launch("data_gemm_kernel");
  if (rc || a.splits == 1) return rc;
  const long long numel = (long long)a.N * a.K * a.L;
  // split_sum's per-channel scale index i / K: K = numel makes it per tensor
  return launch_split_sum(a.partials, a.splits, numel, (int)numel, a.mask, a.scale, a.out,
                          stream);
}

template <int BM, int BN, bool VA, typename T>
static void launch_weight(const float* go, const T* img, atx_conv_geom g, int O, int K, int L,
                          int P, int chunk, int S, int offset, int pad_index,
                          const float* pad_dev, const float* tw, const float* go_sx,
                          const float* go_sw, float* ws, hipStream_t stream) {
  WeightA<BM, VA> la{};
  la.O = O; la.L = L;
  WeightB<BN, T> lb{};
  lb.img = img; lb.g = g; lb.K = K; lb.L = L; lb.offset = offset; lb.pad = pad_index;
  WeightOut ep{ws, O, K, (long long)O * K, go_sx, go_sw};
  dim3 grid((unsigned)cdiv(K, BN), (unsigned)cdiv(O, BM), (unsigned)S);
  hipLaunchKernelGGL((weight_gemm_kernel<BM, BN, VA, WeightB<BN, T>>), grid, dim3(GT), 0,
                     stream, la, lb, ep, go, (long long)P * O, tw, pad_dev, P, chunk);
}

template <bool VA, typename T>
static void dispatch_weight_tiles(const float* go, const T* img, atx_conv_geom g, int O, int K,
                                  int L, int P, int chunk, int S, int offset, int pad_index,
                                  const float* pad_dev, const float* tw, const float* go_sx,
                                  const float* go_sw, float* ws, hipStream_t stream) {
  const int bm = tile_of(O), bn = tile_of(K);
#define ATX_LW(M_, N_)                                                                       \
  launch_weight<M_, N_, VA, T>(go, img, g, O, K, L, P, chunk, S, offset, pad_index, pad_dev, \
                               tw, go_sx, go_sw, ws, stream)
  if (bm == 64 && bn == 64) ATX_LW(64, 64);
  else if (bm == 64) ATX_LW(64, 128);
  else if (bn == 64) ATX_LW(128, 64);
  else ATX_LW(128, 128);
#undef ATX_LW
}

template <typename T>
static void dispatch_weight(const float* go, const T* img, atx_conv_geom g, int O, int K, int L,
                            int P, int chunk, int S, int offset, int pad_index,
                            const float* pad_dev, const float* tw, const float* go_sx,
                            const float* go_sw, float* ws, hipStream_t stream) {
  if (L % 4 == 0 && (uintptr_t)go % 16 == 0)
    dispatch_weight_tiles<true, T>(go, img, g, O, K, L, P, chunk, S, offset, pad_index, pad_dev,
                                   tw, go_sx, go_sw, ws, stream);
  else
    dispatch_weight_tiles<false, T>(go, img, g, O, K, L, P, chunk, S, offset, pad_index,
                                    pad_dev, tw, go_sx, go_sw, ws, stream);
}

template <int BM, int BN, bool VA>
static void launch_weight_rows(const float* go, const uint16_t* xt, long long Rpad, int O,
                               int K, int L, int P, int chunk, int S, const float* tw,
                               const float* go_sx, const float* go_sw, float* ws,
                               hipStream_t stream) {
  WeightA<BM, VA> la{};
  la.O = O; la.L = L;
  WeightBRows<BN> lb{};
  lb.xt = xt; lb.Rpad = Rpad; lb.K = K; lb.Kpad = (K + 3) & ~3;
  WeightOut ep{ws, O, K, (long long)O * K, go_sx, go_sw};
  dim3 grid((unsigned)cdiv(K, BN), (unsigned)cdiv(O, BM), (unsigned)S);
  hipLaunchKernelGGL((weight_gemm_kernel<BM, BN, VA, WeightBRows<BN>>), grid, dim3(GT), 0,
                     stream, la, lb, ep, go, (long long)P * O, tw, (const float*)nullptr, P,
                     chunk);
}

template <bool VA>
static void dispatch_weight_rows(const float* go, const uint16_t* xt, long long Rpad, int O,
                                 int K, int L, int P, int chunk, int S, const float* tw,
                                 const float* go_sx, const float* go_sw, float* ws,
                                 hipStream_t stream) {
  const int bm = tile_of(O), bn = tile_of(K);
#define ATX_LWR(M_, N_) \
  launch_weight_rows<M_, N_, VA>(go, xt, Rpad, O, K, L, P, chunk, S, tw, go_sx, go_sw, ws, stream)
  if (bm == 64 && bn == 64) ATX_LWR(64, 64);
  else if (bm == 64) ATX_LWR(64, 128);
  else if (bn == 64) ATX_LWR(128, 64);
  else ATX_LWR(128, 128);
#undef ATX_LWR
}

template <int BM, bool SC>
static int launch_dgrad(const float* go, const uint8_t* wq, const float* tx,
                        const atx_conv_geom& g, int O, const float* sx, const float* sw,
                        const uint8_t* mask, const float* scale, float* gx, uint16_t* planes,
                        hipStream_t stream) {
  constexpr int BN = 128;
  const int KK = g.KH * g.KW, K = g.C * KK, HW = g.H * g.W, NHW = g.N * HW;
  const bool vo = HW % 4 == 0 && (uintptr_t)gx % 16 == 0 && (uintptr_t)mask % 4 == 0;
  if (planes && planes_fit(HW, O, (long long)g.OH * g.OW)) {
    int rc = launch_weight_planes(wq, tx, O, K, planes, stream);
    if (rc) return rc;
    PlaneA<BM, true> la{};
    la.planes = planes; la.pbytes = (int)weight_planes_bytes(K, O);
    la.Kp = (int)(cdiv(K, 128) * 128); la.Opad = O; la.KK = KK; la.O = O;
    ShiftCols<BN, SC> lb{};
    lb.g = g; lb.O = O; lb.sx = sx; lb.sw = sw;
    DataOut ep{gx, g.C, HW, NHW, mask, scale, 0};
    dim3 grid((unsigned)cdiv(NHW, BN), (unsigned)cdiv(g.C, BM), 1);
    const long long go_elems = (long long)g.N * O * g.OH * g.OW;
    if (vo)
      hipLaunchKernelGGL((dgrad_planes_kernel<BM, SC, true>), grid, dim3(GT), 0, stream, la, lb,
                         ep, go, go_elems, tx, KK * O);
    else
      hipLaunchKernelGGL((dgrad_planes_kernel<BM, SC, false>), grid, dim3(GT), 0, stream, la,
                         lb, ep, go, go_elems, tx, KK * O);
    return check_launch("dgrad_planes_kernel");
  }
  DgradA<BM> la{};
  la.wq = wq; la.K = K; la.KK = KK; la.C = g.C; la.O = O;
  DgradB<BN, SC> lb{};
  lb.go = go; lb.g = g; lb.O = O; lb.NHW = NHW; lb.sx = sx; lb.sw = sw;
  DataOut ep{gx, g.C, HW, NHW, mask, scale, 0};
  dim3 grid((unsigned)cdiv(NHW, BN), (unsigned)cdiv(g.C, BM), 1);
  if (vo)
    hipLaunchKernelGGL((dgrad_gemm_kernel<BM, BN, SC, true>), grid, dim3(GT), 0, stream, la, lb,
                       ep, tx, KK * O);
  else
    hipLaunchKernelGGL((dgrad_gemm_kernel<BM, BN, SC, false>), grid, dim3(GT), 0, stream, la,
                       lb, ep, tx, KK * O);
  return check_launch("dgrad_gemm_kernel");
}

// The implicit backward-data GEMM serves stride-1 convs whose O fills whole
// k-tiles (one tap per tile) and whose C x N*H*W output tiles fill the GPU
// (>= 512 blocks); 1x1 unpadded convs take the direct path.  With fewer
// tiles the col GEMM (M = C*KH*KW) plus col2im is faster: measured on the
// ResNet-50 3x3 layers at batch 64, a split implicit GEMM took 241 us where
// the col path takes 198 us (14x14) and 214 us (7x7); at 28x28 (392 tiles)
// the implicit GEMM takes 255 us against 221 us; at 56x56 the unsplit
// implicit GEMM takes 262-290 us against 462 us.
static bool implicit_dgrad(const atx_conv_geom& g, int O) {
  const long long tiles = cdiv((long long)g.N * g.H * g.W, 128) * cdiv(g.C, tile_of(g.C));
  return g.SH == 1 && g.SW == 1 && O % BK == 0 && O > 0 && tiles >= 512 &&
         !(g.KH == 1 && g.KW == 1 && g.PH == 0 && g.PW == 0) &&
         (long long)g.N * g.C * g.H * g.W < 0x7fffffffLL &&
         (long long)g.KH * g.KW * O < 0x7fffffffLL;
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
    return launch_split_sum(nullptr, 0, (long long)N * K * L, K, nullptr, nullptr, col, stream);
  }
  ATX_REQUIRE(go && wq && tx, "atx_conv_bwd_data_col: null pointer");
  ATX_REQUIRE((long long)N * L < 0x7fffffffLL && cdiv(K, 64) <= 65535,
              "atx_conv_bwd_data_col: sizes too large");
  // no workspace here: the fp32 kernels (table lookups in the loaders)
  const DataArgs a{go, wq, tx, N, O, K, L, nullptr, nullptr, col, nullptr, nullptr, 1, 0,
                   nullptr, nullptr};
  return run_data_gemm(a, stream);
}

// A 1x1, stride-1, unpadded conv's columns are its image gradient.
static bool direct_columns(const atx_conv_geom& g) {
  return g.KH == 1 && g.KW == 1 && g.SH == 1 && g.SW == 1 && g.PH == 0 && g.PW == 0;
}

// Workspace of atx_conv_bwd_data: [bf16 weight planes][split partials][col
// (unless direct or implicit)].
long long atx_conv_bwd_data_workspace_bytes(atx_conv_geom g, int O) {
  const int K = g.C * g.KH * g.KW, L = g.OH * g.OW;
  if (g.N <= 0 || K <= 0 || L <= 0 || O <= 0) return 0;
  const long long planes = weight_planes_bytes(K, O);
  if (implicit_dgrad(g, O)) return planes;
  const long long numel = (long long)g.N * K * L;
  const int S = data_splits(g.N, O, K, L);
  return planes + ((S > 1 ? S : 0) + (direct_columns(g) ? 0 : 1)) * numel * 4;
}

int atx_conv_bwd_data(const float* go, const uint8_t* wq, const float* tx, atx_conv_geom g,
                      int O, const float* go_sx, const float* go_sw, const uint8_t* mask,
                      const float* scale, float* gx, float* workspace, hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && g.N >= 0 && g.C >= 0 && g.H >= 0 && g.W >= 0 && g.KH > 0 && g.KW > 0,
              "atx_conv_bwd_data: bad geometry");
  ATX_REQUIRE((go_sx == nullptr) == (go_sw == nullptr),
              "atx_conv_bwd_data: go_sx and go_sw come together");
  ATX_REQUIRE(!mask || scale, "atx_conv_bwd_data: mask needs scale");
  const long long img = (long long)g.N * g.C * g.H * g.W;
  if (img == 0) return ATX_OK;
  ATX_REQUIRE(gx, "atx_conv_bwd_data: null output");
  const int K = g.C * g.KH * g.KW;
  const int L = g.OH * g.OW;
  // the bf16 weight planes lead the workspace (absent when O, K or L is 0)
  uint16_t* planes = nullptr;
  float* rest = workspace;
  if (O > 0 && K > 0 && L > 0) {
    ATX_REQUIRE(workspace, "atx_conv_bwd_data: null workspace");
    planes = (uint16_t*)workspace;
    rest = (float*)((char*)workspace + weight_planes_bytes(K, O));
  }
  if (L > 0 && implicit_dgrad(g, O)) {
    ATX_REQUIRE(go && wq && tx, "atx_conv_bwd_data: null pointer");
    ATX_REQUIRE(cdiv(g.C, 64) <= 65535, "atx_conv_bwd_data: too many channels");
    const bool sc = go_sw != nullptr;
#define ATX_LD(M_, S_) \
  launch_dgrad<M_, S_>(go, wq, tx, g, O, go_sx, go_sw, mask, scale, gx, planes, stream)
    if (tile_of(g.C) == 64) return sc ? ATX_LD(64, true) : ATX_LD(64, false);
    return sc ? ATX_LD(128, true) : ATX_LD(128, false);
#undef ATX_LD
  }
  const long long numel = (long long)g.N * K * L;
  const int S = (O > 0 && numel > 0) ? data_splits(g.N, O, K, L) : 1;
  float* partials = S > 1 ? rest : nullptr;
  float* col = rest ? rest + (S > 1 ? S * numel : 0) : nullptr;
  ATX_REQUIRE(S == 1 || rest, "atx_conv_bwd_data: null workspace");
  if (direct_columns(g)) {
    if (O == 0 || L == 0)
      return launch_split_sum(nullptr, 0, img, 1, nullptr, nullptr, gx, stream);
    ATX_REQUIRE(go && wq && tx, "atx_conv_bwd_data: null pointer");
    ATX_REQUIRE((long long)g.N * L < 0x7fffffffLL && cdiv(K, 64) <= 65535,
                "atx_conv_bwd_data: sizes too large");
    const DataArgs a{go, wq, tx, g.N, O, K, L, go_sx, go_sw, gx, mask, scale, S, 0, partials,
                     planes};
    return run_data_gemm(a, stream);
  }
  ATX_REQUIRE(rest, "atx_conv_bwd_data: null workspace");
  if ((long long)K * L == 0 || O == 0) {
    if (numel) {
      int rc = launch_split_sum(nullptr, 0, numel, 1, nullptr, nullptr, col, stream);
      if (rc) return rc;
    }
  } else {
    ATX_REQUIRE(go && wq && tx, "atx_conv_bwd_data: null pointer");
    ATX_REQUIRE((long long)g.N * L < 0x7fffffffLL && cdiv(K, 64) <= 65535,
                "atx_conv_bwd_data: sizes too large");
    const DataArgs a{go, wq, tx, g.N, O, K, L, go_sx, go_sw, col, nullptr, nullptr, S, 0,
                     partials, planes};
    int rc = run_data_gemm(a, stream);
    if (rc) return rc;
  }
  return atx_col2im(col, g, mask, scale, gx, stream);
}

long long atx_conv_bwd_weight_workspace_bytes(int O, int K, long long P) {
  if (O <= 0 || K <= 0 || P <= 0) return 0;
  return (long long)weight_splits(O, K, P) * O * K * 4;
}

int atx_conv_bwd_weight(const float* go, const void* img, int dtype, atx_conv_geom g, int O,
                        int pad_index, const float* pad_dev, const float* tw,
                        const float* go_sx, const float* go_sw,
                        const uint8_t* mask_w, const float* scale_w, float* gw,
                        float* workspace, hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && dtype >= 0 && dtype <= 3, "atx_conv_bwd_weight: bad arguments");
  ATX_REQUIRE((go_sx == nullptr) == (go_sw == nullptr),
              "atx_conv_bwd_weight: go_sx and go_sw come together");
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
    return launch_split_sum(nullptr, 0, (long long)O * K, K, nullptr, scale_w, gw, stream);
  }
  ATX_REQUIRE(go && img && workspace, "atx_conv_bwd_weight: null operand/workspace");
  ATX_REQUIRE(cdiv(O, 64) <= 65535, "atx_conv_bwd_weight: too many output channels");
  ATX_REQUIRE((long long)O * L < (1LL << 28), "%s: one image's output gradient exceeds 1 GiB",
              __func__);
  const int S = weight_splits(O, K, P);
  const int chunk = (int)(cdiv(cdiv(P, S), BK) * BK);
  const int Sreal = (int)cdiv(P, chunk);
  if (dtype == 0)
    dispatch_weight<int8_t>(go, (const int8_t*)img, g, O, K, L, (int)P, chunk, Sreal, 128,
                            pad_index, pad_dev, tw, go_sx, go_sw, workspace, stream);
  else if (dtype == 1)
    dispatch_weight<uint8_t>(go, (const uint8_t*)img, g, O, K, L, (int)P, chunk, Sreal, 0,
                             pad_index, pad_dev, tw, go_sx, go_sw, workspace, stream);
  else
    dispatch_weight<float>(go, (const float*)img, g, O, K, L, (int)P, chunk, Sreal,
                           f32_offset, pad_index, pad_dev, tw, go_sx, go_sw, workspace, stream);
  int rc = check_launch("weight_gemm_kernel");
  if (rc) return rc;
  return launch_split_sum(workspace, Sreal, (long long)O * K, K, mask_w, scale_w, gw, stream);
}

int atx_conv_bwd_weight_rows(const float* go, const uint16_t* xt, int Rpad, int N, int K,
                             int L, int O, const float* tw, const float* go_sx,
                             const float* go_sw, const uint8_t* mask_w, const float* scale_w,
                             float* gw, float* workspace, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0 && O >= 0, "atx_conv_bwd_weight_rows: negative size");
  ATX_REQUIRE((go_sx == nullptr) == (go_sw == nullptr),
              "atx_conv_bwd_weight_rows: go_sx and go_sw come together");
  const long long P = (long long)N * L;
  ATX_REQUIRE(P < 0x7fffffffLL, "atx_conv_bwd_weight_rows: N*L too large");
  ATX_REQUIRE(Rpad >= P && Rpad % ATX_ROW_TILE == 0, "atx_conv_bwd_weight_rows: bad Rpad %d",
              Rpad);
  if ((long long)O * K == 0) return ATX_OK;
  ATX_REQUIRE(gw && tw && (!mask_w || scale_w), "atx_conv_bwd_weight_rows: null pointer");
  if (P == 0)
    return launch_split_sum(nullptr, 0, (long long)O * K, K, nullptr, scale_w, gw, stream);
  ATX_REQUIRE(go && xt && workspace, "atx_conv_bwd_weight_rows: null operand/workspace");
  ATX_REQUIRE(cdiv(O, 64) <= 65535, "atx_conv_bwd_weight_rows: too many output channels");
  ATX_REQUIRE((long long)O * L < (1LL << 28), "%s: one image's output gradient exceeds 1 GiB",
              __func__);
  const int S = weight_splits(O, K, P);
  const int chunk = (int)(cdiv(cdiv(P, S), BK) * BK);
  const int Sreal = (int)cdiv(P, chunk);
  if (L % 4 == 0 && (uintptr_t)go % 16 == 0)
    dispatch_weight_rows<true>(go, xt, Rpad, O, K, L, (int)P, chunk, Sreal, tw, go_sx, go_sw,
                               workspace, stream);
  else
    dispatch_weight_rows<false>(go, xt, Rpad, O, K, L, (int)P, chunk, Sreal, tw, go_sx, go_sw,
                                workspace, stream);
  int rc = check_launch("weight_gemm_kernel<rows>");
  if (rc) return rc;
  return launch_split_sum(workspace, Sreal, (long long)O * K, K, mask_w, scale_w, gw, stream);
}

}  // extern "C"
