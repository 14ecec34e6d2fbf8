// grad_x of the pair-table (custom) estimator for weights with at most 16
// distinct indices (weight_bits <= 4), on the bf16 matrix cores:
//   grad_x[n,k,l] = sum_o dy[n,o,l] * DX[xi(n,k,l)][wi(o,k)]
// Reference: csrc/cuda/bgemm_custom_grad_optimize.cu:30-205 (uint8),
// 315-490 (int8); the general pair-table kernel is custom_grad.hip.
//
// With wi(o,k) in [wbase, wbase + 16) the sum regroups by weight index:
//   S[r,k,w] = sum_{o : wi(o,k) = wbase + w} dy[r,o]          (r = n*L + l)
//   grad_x[r,k] = sum_w DX[xi(r,k)][wbase + w] * S[r,k,w]
// S is a dense product dy[R x O] * H_k[O x 16] with the 0/1 matrix
// H_k[o][w] = [wi(o,k) = wbase + w], 16 products per term of the original
// sum, on v_mfma_f32_16x16x32_bf16 (a 16-times larger count of products at
// sixteen times the fp32 FMA rate of the VALU, and no table traffic per term).
// dy is split exactly into three bf16 parts, dy = h + m + l (h = dy with the
// low 16 bits cleared, m likewise of dy - h, l = dy - h - m, each at most 8
// significant bits), so every product part * 1.0 is exact and S is an fp32
// sum of the original terms' parts: its error is that of an fp32 summation,
// bounded by the usual n * eps * sum|terms| of the reference's own order.
//
// Tile: 256 rows x 16 taps per workgroup (8 waves, 32 rows = two 16-row
// blocks each), persistent over the tiles in XCD-contiguous ranges (the 32
// workgroups of an XCD work on consecutive taps of the same rows, so dy comes
// from HBM once per XCD).  For each 32-channel step the waves build the 16
// taps' H fragments in LDS (two taps each, double-buffered, one barrier per
// step) and every wave runs 16 taps x 2 row blocks x 3 parts = 96 MFMAs with
// its own dy parts in registers; D = H^T * dy^T leaves S[w][r] with lane
// (row j = lane % 16, group g = lane / 16) holding w = 4g..4g+3.  The
// epilogue reads the row's table entries DX[xi][wbase + 4g .. +3] (one
// 16-byte LDS read from a 256 x 16 fp32 copy of the table's 16 columns),
// forms the four-term partial sums and adds them over the four lane groups
// with two exchange steps that leave group g with tap 4q + g.
#include "atx_internal.h"

#include <algorithm>

namespace atx {
namespace ohx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int NWAVE = 8;
constexpr int NT = 64 * NWAVE;               // 512 threads
constexpr int RB = 2;                        // 16-row blocks per wave
constexpr int ROWS = NWAVE * RB * 16;        // 256 rows per tile
constexpr int KT = 16;                       // taps per tile
constexpr int OC = 32;                       // channels per MFMA step
constexpr int XS = 80;                       // bytes per table row in LDS (64 + 16 pad)
constexpr int HTAP = 64 * 16;                // bytes of one tap's H fragments
constexpr int HBUF = KT * HTAP;              // one step's H fragments (16 KiB)
constexpr unsigned OOB = 0x80000000u;        // buffer offset past any operand
constexpr int FMAX = 4096;                   // channels with a dy factor (LDS)

struct Params {
  const uint16_t* xt; int Rpad;              // row-offset operand [Kpad][Rpad]
  const uint8_t* wt; int Opad;               // weight indices [K][Opad]
  const float* tab;                          // tab[w * 256 + v] = DX[v][w]
  const float* dy;                           // [N][O][L]
  const float* dys;                          // per-channel factor of dy [O] (nullable)
  float* gx;                                 // [N][K][L]
  // img: grad_x of a 1x1 stride-1 unpadded conv is the image gradient; the
  // epilogue then adds pos[n][l] (nullable) and applies the fake-quant STE
  // (mask nullable, scale with it), atx_col2im_pos's operations for that
  // geometry
  const float* pos; const uint8_t* mask; const float* scale;
  int K, R, L, O, wbase;
  int tiles_k, tiles;
  unsigned dy_bytes, wt_bytes, xt_bytes;
  unsigned pos_bytes, mask_bytes;            // 0 for a null pos / mask
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// H fragment of one tap for lane (w = lane % 16, group g): 8 bytes of weight
// indices (channels ob + 8g + 0..7) -> bf16 1.0 where the index is wbase + w.
// bf16 element 2p holds channel 8g + p, element 2p + 1 channel 8g + 4 + p
// (the same order the dy parts use).  `keep` masks the bytes of channels at
// or past O.
__device__ __forceinline__ u32x4 h_fragment(uint2 b, unsigned brep, unsigned wrep,
                                            uint2 keep) {
  const unsigned x0 = (b.x - brep) ^ wrep, x1 = (b.y - brep) ^ wrep;
  // index bytes lie in [wbase, wbase + 16): x bytes in [0, 16), 0x80 where 0
  const unsigned e0 = (0x80808080u - x0) & 0x80808080u & keep.x;
  const unsigned e1 = (0x80808080u - x1) & 0x80808080u & keep.y;
  u32x4 f;
#pragma unroll
  for (int p = 0; p < 4; ++p)   // [e0 byte p, 0, e1 byte p, 0] * 0x7f -> 0x3f80 halves
    f[p] = __umul24(__builtin_amdgcn_perm(e1, e0, 0x0C040C00u + 0x00010001u * p), 0x7fu);
  return f;
}

// Byte mask of the first n bytes (n clamped to 0..4).
__device__ __forceinline__ unsigned byte_mask(int n) {
  return n >= 4 ? 0xffffffffu : (n <= 0 ? 0u : (1u << (8 * n)) - 1u);
}

// The three bf16 parts of eight dy values (channels 8g + 0..7) in MFMA
// operand order: part dword p = [value p, value 4 + p] truncated to bf16.
__device__ __forceinline__ void split_parts(const float (&d)[8], u32x4 (&P)[3]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const unsigned a = __float_as_uint(d[p]), b = __float_as_uint(d[4 + p]);
    P[0][p] = __builtin_amdgcn_perm(b, a, 0x07060302u);
    const float ra = bf16_rest(d[p]);
    const float rb = bf16_rest(d[4 + p]);
    const unsigned ua = __float_as_uint(ra), ub = __float_as_uint(rb);
    P[1][p] = __builtin_amdgcn_perm(ub, ua, 0x07060302u);
    const float la = ra - __uint_as_float(ua & 0xffff0000u);
    const float lb = rb - __uint_as_float(ub & 0xffff0000u);
    P[2][p] = __builtin_amdgcn_perm(__float_as_uint(lb), __float_as_uint(la), 0x07060302u);
  }
}

template <bool IMG>
__global__ void __launch_bounds__(NT, 1) onehot_dx_kernel(const Params p) {
  __shared__ __align__(16) unsigned char hbuf[2 * HBUF];
  __shared__ __align__(16) unsigned char xtab[256 * XS];
  // the epilogue's row offsets, per wave: 16 operand slots x 32 rows
  __shared__ __align__(16) uint16_t xsh[NWAVE][KT][RB * 16];
  // dy's per-channel factors (zero past O)
  __shared__ __align__(16) float fsh[FMAX];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, j = lane & 15;
  const int nsteps = (p.O + OC - 1) / OC;

  // the table's 16 columns wbase .. wbase + 15 as rows of 16 fp32
  for (int e = tid; e < 256 * 16; e += NT) {
    const int w = e >> 8, v = e & 255;
    *(float*)(xtab + v * XS + w * 4) = p.tab[(p.wbase + w) * 256 + v];
  }
  if (p.dys)
    for (int e = tid; e < nsteps * OC; e += NT) fsh[e] = e < p.O ? p.dys[e] : 0.f;

  const __amdgpu_buffer_rsrc_t dyr = rsrc(p.dy, p.dy_bytes);
  const __amdgpu_buffer_rsrc_t wtr = rsrc(p.wt, p.wt_bytes);
  const __amdgpu_buffer_rsrc_t xtr = rsrc(p.xt, p.xt_bytes);
  const unsigned wrep = (unsigned)j * 0x01010101u;
  const unsigned brep = (unsigned)p.wbase * 0x01010101u;
  const int chan_bytes = p.L * 4;
  const int ptail = p.O - (nsteps - 1) * OC;           // channels of the last step
  // The image epilogue's operands: range-checked loads (a null operand has
  // no bytes, its loads return 0) and, for a null one, a value that leaves the
  // sum as it is: -0 for the position term, 1 for every mask byte, 1 for the
  // STE divisor (read once: the epilogue's stores may alias p.scale).
  const __amdgpu_buffer_rsrc_t posr = rsrc(p.pos ? (const void*)p.pos : p.gx, p.pos_bytes);
  const __amdgpu_buffer_rsrc_t mkr = rsrc(p.mask ? (const void*)p.mask : p.gx, p.mask_bytes);
  const unsigned pos_fill = p.pos ? 0u : 0x80000000u;
  const unsigned mk_fill = p.mask ? 0u : 1u;
  const float sdiv = (IMG && p.mask) ? fmaxf(p.scale[0], 1e-12f) : 1.0f;

  // Persistent over the tiles (each XCD walks a contiguous range), one
  // pipeline across tile boundaries: the last channel step of a tile
  // prefetches the next tile's first dy block and index bytes and builds its
  // first H fragments, so a tile starts with its operands in place.
  const int nb = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, bslot = bid >> 3, per = nb >> 3;   // nb is a multiple of 8
  auto tile_at = [&](int it) { return (long long)it * nb + xcd * per + bslot; };

  // per-tile operand addresses of this lane
  struct Where { int rt, k0, kh0, kh1; unsigned dyoff[RB]; };
  auto where = [&](int tile, Where& w) {
    w.rt = tile / p.tiles_k;
    w.k0 = (tile - w.rt * p.tiles_k) * KT;
    // this wave's two taps of H (indices of tap k >= K are never stored)
    w.kh0 = std::min(w.k0 + 2 * wave, p.K - 1);
    w.kh1 = std::min(w.k0 + 2 * wave + 1, p.K - 1);
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const int r = w.rt * ROWS + wave * (RB * 16) + b * 16 + j;
      const int n = r / p.L, l = r - n * p.L;
      w.dyoff[b] = r < p.R ? (unsigned)((((long long)n * p.O + 8 * g) * p.L + l) * 4) : OOB;
    }
  };
  auto load_w = [&](const Where& w, int s, uint2 (&wv)[2]) {
    const int ob = s * OC + 8 * g;
    wv[0] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                          wtr, ob, w.kh0 * p.Opad, 0));
    wv[1] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                          wtr, ob, w.kh1 * p.Opad, 0));
  };
  auto load_dy = [&](const Where& w, int s, float (&d)[RB][8]) {
    const int nvalid = s == nsteps - 1 ? ptail - 8 * g : 8;   // channels below O
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
      for (int c = 0; c < 8; ++c)
        d[b][c] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(
                       dyr, c < nvalid ? w.dyoff[b] : OOB, (s * OC + c) * chan_bytes, 0));
  };
  auto write_h = [&](int s, const uint2 (&wv)[2], int buf) {
    uint2 keep = {0xffffffffu, 0xffffffffu};
    if (s == nsteps - 1) {
      const int nv = ptail - 8 * g;
      keep = {byte_mask(nv), byte_mask(nv - 4)};
    }
    unsigned char* dst = hbuf + buf * HBUF + (2 * wave) * HTAP + lane * 16;
    *(u32x4*)dst = h_fragment(wv[0], brep, wrep, keep);
    *(u32x4*)(dst + HTAP) = h_fragment(wv[1], brep, wrep, keep);
  };

  int it = 0;
  if (tile_at(0) >= p.tiles) return;           // every wave of the workgroup alike
  Where cur, nxt;
  where((int)tile_at(0), cur);
  float raw[RB][8];
  {
    uint2 w0[2];
    load_w(cur, 0, w0);
    load_dy(cur, 0, raw);
    write_h(0, w0, 0);
  }
  __syncthreads();
  int hsel = 0;

  for (;;) {
    const long long ln = tile_at(it + 1);
    const bool has_next = ln < p.tiles;
    if (has_next) where((int)ln, nxt);
    f32x4 acc[RB][KT];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
      for (int t = 0; t < KT; ++t) acc[b][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 xq = {0u, 0u, 0u, 0u};

    for (int s = 0; s < nsteps; ++s) {
      if (p.dys) {            // dy * factor[o], the product the caller would form
        const float4 f0 = *(const float4*)&fsh[s * OC + 8 * g];
        const float4 f1 = *(const float4*)&fsh[s * OC + 8 * g + 4];
        const float f[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
        for (int b = 0; b < RB; ++b)
#pragma unroll
          for (int c = 0; c < 8; ++c) raw[b][c] *= f[c];
      }
      u32x4 P[RB][3];
#pragma unroll
      for (int b = 0; b < RB; ++b) split_parts(raw[b], P[b]);
      const bool last = s + 1 == nsteps;
      uint2 wn[2];
      if (!last) {
        load_w(cur, s + 1, wn);
        load_dy(cur, s + 1, raw);
      } else {
        // row offsets of the tile's 16 slots for the wave's 32 rows: lane l
        // loads slot l / 4, rows 8 (l % 4) .. + 7 (slots past K read 0)
        const unsigned xq_off =
            ((unsigned)(cur.k0 + (lane >> 2)) * (unsigned)p.Rpad +
             (unsigned)(cur.rt * ROWS + wave * (RB * 16) + 8 * (lane & 3))) * 2u;
        xq = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xtr, xq_off, 0, 0));
        if (has_next) {
          load_w(nxt, 0, wn);
          load_dy(nxt, 0, raw);
        }
      }
      // H fragments of tap quad tq + 1 are read while quad tq's MFMAs issue
      const unsigned char* hb = hbuf + hsel * HBUF + lane * 16;
      u32x4 H[2][4];
#pragma unroll
      for (int t = 0; t < 4; ++t) H[0][t] = *(const u32x4*)(hb + t * HTAP);
#pragma unroll
      for (int tq = 0; tq < KT / 4; ++tq) {
        if (tq + 1 < KT / 4) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            H[(tq + 1) & 1][t] = *(const u32x4*)(hb + (4 * (tq + 1) + t) * HTAP);
        }
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int b = 0; b < RB; ++b)
              acc[b][4 * tq + t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bf16x8, H[tq & 1][t]), __builtin_bit_cast(bf16x8, P[b][q]),
                  acc[b][4 * tq + t], 0, 0, 0);
      }
      if (!last) write_h(s + 1, wn, hsel ^ 1);
      else if (has_next) write_h(0, wn, hsel ^ 1);
      __syncthreads();
      hsel ^= 1;
    }

    // epilogue: grad_x[r, k] = sum_w DX[xi(r,k)][wbase + w] * S[w][r]
    *(uint4*)&xsh[wave][lane >> 2][8 * (lane & 3)] = xq;
    __builtin_amdgcn_wave_barrier();          // the wave's own rows: no workgroup barrier
    asm volatile("" ::: "memory");
    // the image epilogue's position terms and STE mask bytes of this lane's
    // rows and taps, loaded before its first store so that no load waits on
    // a store (registers are free here; in the product steps they are not)
    float posv[RB];
    unsigned mk[RB][KT / 4];
    if constexpr (IMG) {
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int r = cur.rt * ROWS + wave * (RB * 16) + b * 16 + j;
        const int n = r / p.L, l = r - n * p.L;
        const bool rvalid = r < p.R;
        const float pv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                       posr, rvalid ? (unsigned)r * 4u : OOB, 0, 0));
        posv[b] = __uint_as_float(__float_as_uint(0.0f + pv) | pos_fill);
        const unsigned mbase = (unsigned)n * (unsigned)p.K * (unsigned)p.L + (unsigned)l;
#pragma unroll
        for (int tq = 0; tq < KT / 4; ++tq) {
          const int k = cur.k0 + 4 * tq + g;
          mk[b][tq] = __builtin_amdgcn_raw_buffer_load_b8(
                          mkr, rvalid && k < p.K ? mbase + (unsigned)k * (unsigned)p.L : OOB, 0, 0) |
                      mk_fill;
        }
      }
    }
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const int r = cur.rt * ROWS + wave * (RB * 16) + b * 16 + j;
      const int n = r / p.L, l = r - n * p.L;
      const bool rvalid = r < p.R;
      const long long gbase = (long long)n * p.K * p.L + l;
      unsigned xo[KT];
#pragma unroll
      for (int t = 0; t < KT; ++t)            // slot of tap k0 + t for row r (k0 % 4 == 0)
        xo[t] = xsh[wave][(t & ~3) | ((t - (r >> 2)) & 3)][b * 16 + j];
#pragma unroll
      for (int tq = 0; tq < KT / 4; ++tq) {
        float part[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const f32x4 e = *(const f32x4*)(xtab + (xo[4 * tq + u] >> 8) * XS + g * 16);
          const f32x4 a = acc[b][4 * tq + u];
          float v = e[0] * a[0];
          v = __builtin_fmaf(e[1], a[1], v);
          v = __builtin_fmaf(e[2], a[2], v);
          v = __builtin_fmaf(e[3], a[3], v);
          part[u] = v;
        }
        // groups {g, g^2} keep taps {0,1} (g < 2) or {2,3}, then {g, g^1}
        const bool hi = g & 2, lo = g & 1;
        const float s0 = hi ? part[0] : part[2], s1 = hi ? part[1] : part[3];
        const float k0v = hi ? part[2] : part[0], k1v = hi ? part[3] : part[1];
        const float q0 = k0v + __shfl_xor(s0, 32), q1 = k1v + __shfl_xor(s1, 32);
        const float sx = lo ? q0 : q1, kx = lo ? q1 : q0;
        const float tot = kx + __shfl_xor(sx, 16);
        const int k = cur.k0 + 4 * tq + g;
        if (rvalid && k < p.K) {
          const long long i = gbase + (long long)k * p.L;
          float v = tot;
          if constexpr (IMG) {    // the col2im sum of one tap, in its order
            v = 0.0f + tot + posv[b];
            v = (mk[b][tq] ? v : 0.0f) / sdiv;
          }
          p.gx[i] = v;
        }
      }
    }
    if (!has_next) break;
    cur = nxt;
    ++it;
  }
}

// The image gradient of a 1x1 stride-1 conv with no output channels: the
// epilogue's operations on a zero sum.
__global__ void img_empty_kernel(int N, int K, int L, const float* __restrict__ pos,
                                 const uint8_t* __restrict__ mask,
                                 const float* __restrict__ scale, float* __restrict__ img) {
  const long long total = (long long)N * K * L;
  const float s = mask ? fmaxf(scale[0], 1e-12f) : 1.0f;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    float v = 0.0f + 0.0f;
    if (pos) {
      const long long n = i / ((long long)K * L), l = i % L;
      v += 0.0f + pos[n * L + l];
    }
    if (mask) v = (mask[i] ? v : 0.0f) / s;
    img[i] = v;
  }
}

}  // namespace ohx
}  // namespace atx

using namespace atx;

static int custom_dx_narrow(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                            const float* dy, const float* dy_scale, const float* tabT, int wbase,
                            int N, int K, int L, int O, const float* pos, const uint8_t* mask,
                            const float* scale, int img, float* grad_x, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0 && O >= 0, "atx_custom_grad_dx_narrow: negative size");
  ATX_REQUIRE(wbase >= 0 && wbase <= 240, "atx_custom_grad_dx_narrow: wbase must be in [0, 240]");
  ATX_REQUIRE(!mask || scale, "atx_custom_grad_dx_narrow_img: mask without scale");
  const long long R = (long long)N * L;
  const long long numel = R * K;
  if (numel == 0) return ATX_OK;
  if (O == 0 && !img)   // an empty sum: zeros
    return atx_custom_grad_dx(xt, Rpad, wt, Opad, dy, tabT, N, K, L, O, grad_x, stream);
  if (O == 0) {         // an empty sum with the position term and the STE
    ATX_REQUIRE(grad_x, "atx_custom_grad_dx_narrow_img: null output");
    hipLaunchKernelGGL(ohx::img_empty_kernel, dim3(elem_grid(numel, 256)), dim3(256), 0, stream,
                       N, K, L, pos, mask, scale, grad_x);
    return check_launch("img_empty_kernel");
  }
  ATX_REQUIRE(xt && wt && dy && tabT && grad_x, "atx_custom_grad_dx_narrow: null pointer");
  ATX_REQUIRE(Rpad >= R && Rpad % ATX_ROW_TILE == 0,
              "atx_custom_grad_dx_narrow: Rpad must be a multiple of %d and >= N*L",
              ATX_ROW_TILE);
  ATX_REQUIRE(Opad >= O && Opad % 32 == 0, "atx_custom_grad_dx_narrow: Opad must be a multiple of 32 and >= O");
  ATX_REQUIRE(!dy_scale || O <= ohx::FMAX,
              "atx_custom_grad_dx_narrow: dy_scale supports at most %d channels", ohx::FMAX);
  ATX_REQUIRE(R * O * 4 < 0x7fffffffLL && (long long)K * Opad < 0x7fffffffLL &&
                  (long long)operand_rows(K) * Rpad * 2 < 0x7fffffffLL,
              "atx_custom_grad_dx_narrow: operand too large for 32-bit buffer offsets");
  ohx::Params p{};
  p.xt = xt; p.Rpad = Rpad; p.wt = wt; p.Opad = Opad; p.tab = tabT; p.dy = dy; p.gx = grad_x;
  p.dys = dy_scale;
  p.pos = pos; p.mask = mask; p.scale = scale;
  p.K = K; p.R = (int)R; p.L = L; p.O = O; p.wbase = wbase;
  p.tiles_k = (int)cdiv(K, ohx::KT);
  const long long tiles = cdiv(R, ohx::ROWS) * p.tiles_k;
  ATX_REQUIRE(tiles < 0x7fffffffLL, "atx_custom_grad_dx_narrow: grid too large");
  p.tiles = (int)tiles;
  p.dy_bytes = (unsigned)(R * O * 4);
  p.wt_bytes = (unsigned)((long long)K * Opad);
  p.xt_bytes = (unsigned)((long long)operand_rows(K) * Rpad * 2);
  ATX_REQUIRE(!img || numel < 0x7fffffffLL,
              "atx_custom_grad_dx_narrow_img: image too large for 32-bit buffer offsets");
  p.pos_bytes = pos ? (unsigned)(R * 4) : 0u;
  p.mask_bytes = mask ? (unsigned)numel : 0u;
  // one workgroup per CU (512 threads at up to 256 registers), a multiple of
  // the 8 XCDs
  const int blocks = (int)std::min<long long>(256, ((tiles + 7) / 8) * 8);
  if (img)
    hipLaunchKernelGGL(ohx::onehot_dx_kernel<true>, dim3(blocks), dim3(ohx::NT), 0, stream, p);
  else
    hipLaunchKernelGGL(ohx::onehot_dx_kernel<false>, dim3(blocks), dim3(ohx::NT), 0, stream, p);
  return check_launch("onehot_dx_kernel");
}

extern "C" {

int atx_custom_grad_dx_narrow(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                              const float* dy, const float* dy_scale, const float* tabT,
                              int wbase, int N, int K, int L, int O, float* grad_x,
                              hipStream_t stream) {
  return custom_dx_narrow(xt, Rpad, wt, Opad, dy, dy_scale, tabT, wbase, N, K, L, O, nullptr,
                          nullptr, nullptr, 0, grad_x, stream);
}

int atx_custom_grad_dx_narrow_img(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                                  const float* dy, const float* dy_scale, const float* tabT,
                                  int wbase, int N, int K, int L, int O, const float* pos,
                                  const uint8_t* mask, const float* scale, float* grad_img,
                                  hipStream_t stream) {
  return custom_dx_narrow(xt, Rpad, wt, Opad, dy, dy_scale, tabT, wbase, N, K, L, O, pos, mask,
                          scale, 1, grad_img, stream);
}

}  // extern "C"
