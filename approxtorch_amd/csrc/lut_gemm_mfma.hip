// LUT GEMM for weights with at most 16 distinct indices (weight_bits <= 4),
// on the int8 matrix cores:
//   y[r, o] = sum_k LUT[xi(r,k)][wi(o,k)]           (r = n*L + l, exact int32)
// Reference: csrc/claude/bgemm_lut_kernels.cuh:183-387 (the tiled integer
// LUT GEMM); the general kernel is lut_gemm.hip.
//
// With wi(o,k) in [wbase, wbase + 16) the sum regroups over (k, w):
//   y[r, o] = sum_{k,w} G[r,(k,w)] * H[(k,w), o],
//   G[r,(k,w)] = LUT[xi(r,k)][wbase + w],  H[(k,w), o] = [wi(o,k) = wbase + w],
// a dense product with a 0/1 right operand.  The 16-bit entries are split
// into two int8 planes (high byte, low byte - 128; for unsigned tables the
// high byte - 128 as well), each plane one v_mfma_i32_16x16x64_i8 per 16 x 16
// block and tap quad (64 = 4 taps x 16 indices), and recombined exactly:
//   y = 256 * D_hi + D_lo + c * K_valid,  c = 128 (int16), 128 * 257 (uint16)
// (every valid tap has exactly one index match in H).  32 int8 products per
// LUT term at the int8 rate of 5 POP/s bound the kernel at 78.6 T LUT-MAC/s,
// twice the VALU bound of the table-gather kernel.
//
// The G operand needs no per-tap table: a lane's 16 bytes of G for one tap
// are row xi of a 256 x 16 byte plane, read with one ds_read_b128.  The
// planes are held in LDS 16 times over (row xi: [plane][copy][16 bytes]), and
// the lane of row m reads copy m, so the 16 lanes of a read pass hit 16
// different bank quads whatever their rows.  H is built per tap quad by the
// eight waves (one 16-channel block each, from one index byte per lane) into
// a double buffer, one barrier per quad.  A workgroup (8 waves) owns 256 rows
// x 128 channels (512 x 64 when O <= 64), a wave 64 rows x 64 channels (4 x 4
// blocks, two planes: 128 int32 accumulators per lane); workgroups are persistent over the tiles
// in XCD-contiguous ranges, and split-K (int32 partial slices, summed by the
// LUT GEMM's split reduce) fills the GPU when the tiles are few.
#include "atx_internal.h"

#include <algorithm>

namespace atx {
namespace ohf {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int NWAVE = 8;
constexpr int NT = 64 * NWAVE;
constexpr int RB = 4, CB = 4;                // 16 x 16 blocks per wave (64 x 64)
constexpr int TROW = 512;                    // LDS bytes per table row: 2 planes x 16 copies x 16
constexpr int TAB = 256 * TROW;              // 128 KiB
constexpr int HBLK = 64 * 16;                // one 16-channel block's H fragments
constexpr int HBUF = 8 * HBLK;               // one quad's H, up to 128 channels (8 KiB)
constexpr int KMAX = 32768;                  // taps per pass with exact int32 sums (uint16)

struct Params {
  const uint16_t* xt; int Rpad;
  const uint8_t* wt; int Opad;
  const uint16_t* lut16t;                    // lut16t[w * 256 + v] = LUT[v][w] (16-bit)
  int K, R, L, O, wbase, is_signed;
  int out_kind;                              // ATX_OUT_* (int32 partials when split)
  void* y;
  const float* sx; const float* sw; const float* bias;
  U8Terms u8;                                // out_kind OUT_DEQUANT_U8
  long long split_stride;                    // elements per partial slice (splits > 1)
  int tiles_r, tiles_c, splits, kq;          // kq = tap quads per split
  int tiles;
  unsigned xt_bytes, wt_bytes;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// H fragment of lane (channel j, tap group g) from its index byte: byte w of
// the 16 is 1 where the index is wbase + w (none for an index outside).
__device__ __forceinline__ i32x4 h_fragment(unsigned wbyte, int wbase, bool valid) {
  const unsigned w = wbyte - (unsigned)wbase;
  const unsigned bit = 1u << ((w & 3u) * 8u);
  const unsigned d = valid ? (w >> 2) : 4u;
  i32x4 f;
#pragma unroll
  for (int p = 0; p < 4; ++p) f[p] = d == (unsigned)p ? (int)bit : 0;
  return f;
}

// WCN waves along the channels: 2 -> 256 rows x 128 channels per workgroup,
// 1 -> 512 rows x 64 channels (layers with O <= 64).
template <int WCN>
__global__ void __launch_bounds__(NT, 1) onehot_gemm_kernel(const Params p) {
  constexpr int NWR = NWAVE / WCN;
  constexpr int TR = 64 * NWR, TC = 64 * WCN;
  __shared__ __align__(16) unsigned char tab[TAB];
  __shared__ __align__(16) unsigned char hbuf[2 * HBUF];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m = lane & 15, g = lane >> 4;
  const int wr = wave % NWR, wc = wave / NWR;

  // planes of the table's 16 columns, 16 copies each
  {
    const int x = tid >> 1, plane = tid & 1;
    unsigned d[4] = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const unsigned v = p.lut16t[(p.wbase + w) * 256 + x];
      const unsigned b = plane == 0 ? ((v >> 8) & 255u) ^ (p.is_signed ? 0u : 0x80u)
                                    : (v & 255u) ^ 0x80u;
      d[w >> 2] |= b << (8 * (w & 3));
    }
    const uint4 q = make_uint4(d[0], d[1], d[2], d[3]);
#pragma unroll
    for (int c = 0; c < 16; ++c) *(uint4*)(tab + x * TROW + plane * 256 + c * 16) = q;
  }

  const __amdgpu_buffer_rsrc_t xtr = rsrc(p.xt, p.xt_bytes);
  const __amdgpu_buffer_rsrc_t wtr = rsrc(p.wt, p.wt_bytes);
  const int nq = (p.K + 3) >> 2;
  const int corr = p.is_signed ? 128 : 128 * 257;
  // slot of tap 4q + g for the lane's rows (r = 16-aligned base + m): the
  // operand's rotation (g - (r >> 2)) & 3
  const int slot_off = (g - (m >> 2)) & 3;

  const int nb = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, bslot = bid >> 3, per = nb >> 3;   // nb is a multiple of 8
  for (int it = 0;; ++it) {
    const long long lt = (long long)it * nb + xcd * per + bslot;
    if (lt >= p.tiles) break;
    // tile order (row tile, split, channel tile): consecutive tiles share rows
    int t = (int)lt;
    const int ct = t % p.tiles_c; t /= p.tiles_c;
    const int sp = t % p.splits;
    const int rt = t / p.splits;
    const int qa = sp * p.kq, qb = std::min(nq, qa + p.kq);
    const int r0 = rt * TR + wr * 64;          // the wave's first row
    const int c0 = ct * TC + wc * 64;          // the wave's first channel

    // the wave's H block for the workgroup: channels ct*TC + 16*wave + m, tap 4q + g
    const int hch = ct * TC + 16 * wave + m;
    auto load_w = [&](int q) -> unsigned {   // the tap differs per lane group
      const int k = std::min(4 * q + g, p.K - 1);
      return __builtin_amdgcn_raw_buffer_load_b8(wtr, (unsigned)(k * p.Opad + hch), 0, 0);
    };
    const bool builds_h = wave < TC / 16;
    auto write_h = [&](int q, unsigned wbyte) {
      const bool valid = 4 * q + g < p.K;
      if (builds_h)
        *(i32x4*)(hbuf + (q & 1) * HBUF + wave * HBLK + lane * 16) =
            h_fragment(wbyte, p.wbase, valid);
    };
    // row offsets of the lane's four row blocks at quad q (slot 4q + slot_off)
    const unsigned xvoff = (unsigned)(slot_off * p.Rpad + r0 + m) * 2u;
    auto load_x = [&](int q, unsigned (&xo)[RB]) {
#pragma unroll
      for (int b = 0; b < RB; ++b)
        xo[b] = __builtin_amdgcn_raw_buffer_load_b16(xtr, xvoff, (4 * q * p.Rpad + 16 * b) * 2,
                                                      0);
    };

    i32x4 acc[RB][CB][2];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
      for (int c = 0; c < CB; ++c) acc[b][c][0] = acc[b][c][1] = i32x4{0, 0, 0, 0};

    unsigned xo0[RB], xo1[RB];
    unsigned wn = load_w(qa);
    load_x(qa, xo0);
    write_h(qa, wn);
    if (qa + 1 < qb) {
      wn = load_w(qa + 1);
      load_x(qa + 1, xo1);
    }
    __syncthreads();

    for (int q = qa; q < qb; ++q) {
      // G fragments of this quad (rows xi of the planes, copy m)
      i32x4 Ghi[RB], Glo[RB];
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const unsigned a = ((xo0[b] & 0xff00u) << 1) | (unsigned)(m * 16);
        Ghi[b] = *(const i32x4*)(tab + a);
        Glo[b] = *(const i32x4*)(tab + a + 256);
      }
      i32x4 H[CB];
#pragma unroll
      for (int c = 0; c < CB; ++c)
        H[c] = *(const i32x4*)(hbuf + (q & 1) * HBUF + (wc * CB + c) * HBLK + lane * 16);
      // prefetch: offsets and index bytes two quads ahead
#pragma unroll
      for (int b = 0; b < RB; ++b) xo0[b] = xo1[b];
      const unsigned wcur = wn;
      if (q + 2 < qb) {
        wn = load_w(q + 2);
        load_x(q + 2, xo1);
      }
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int b = 0; b < RB; ++b) {
          acc[b][c][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Ghi[b], H[c], acc[b][c][0], 0, 0, 0);
          acc[b][c][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Glo[b], H[c], acc[b][c][1], 0, 0, 0);
        }
      if (q + 1 < qb) write_h(q + 1, wcur);
      __syncthreads();
    }

    // epilogue: lane (channel c0 + 16c + m, group g) holds rows 4g .. 4g + 3 of
    // each row block
    const int kvalid = std::min(p.K, 4 * qb) - 4 * qa;
    const int cK = corr * kvalid;
    const bool split = p.splits > 1;
    const int okind = split ? ATX_OUT_I32 : p.out_kind;
    const long long sbase = split ? (long long)sp * p.split_stride : 0;
    const bool u8 = okind == OUT_DEQUANT_U8;
    const float sx = okind == ATX_OUT_DEQUANT || u8 ? p.sx[0] : 0.f;
    // uint8 correction: the rows' tap sums, read once for all channels
    const float z = u8 ? p.u8.zx[0] : 0.f, kz = p.u8.K * z;
    float xr[RB][4];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xr[b][e] = u8 ? p.u8.xs[std::min(r0 + 16 * b + 4 * g + e, p.R - 1)] : 0.f;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const int o = c0 + 16 * c + m;
      if (o >= p.O) continue;
      float sc = 0.f, bo = 0.f, zo = 0.f, wo = 0.f, ko = 0.f;
      if (okind == ATX_OUT_DEQUANT || u8) {
        sc = sx * p.sw[o];
        bo = p.bias ? p.bias[o] : 0.f;
      }
      if (u8) {
        zo = p.u8.zw[o];
        wo = z * p.u8.ws[o];
        ko = kz * zo;
      }
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int rq = r0 + 16 * b + 4 * g;    // first of four consecutive rows
        if (rq >= p.R) continue;
        int v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)   // exact mod 2^32; the sum itself fits int32
          v[e] = (int)(256u * (unsigned)acc[b][c][0][e] + (unsigned)acc[b][c][1][e] +
                       (unsigned)cK);
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (u8) {
            f[e] = u8_dequant((float)v[e], xr[b][e], zo, wo, ko, sc, p.bias, bo);
          } else if (okind == ATX_OUT_DEQUANT) {
            const float tv = (float)v[e] * sc;
            f[e] = p.bias ? bo + tv : tv;
          } else {
            f[e] = (float)v[e];
          }
        }
        int n = rq / p.L, l = rq - n * p.L;
        if (p.L % 4 == 0 && rq + 3 < p.R) {
          const long long idx = sbase + ((long long)n * p.O + o) * p.L + l;
          if (okind == ATX_OUT_I32)
            *(int4*)((int*)p.y + idx) = make_int4(v[0], v[1], v[2], v[3]);
          else
            *(float4*)((float*)p.y + idx) = make_float4(f[0], f[1], f[2], f[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (rq + e < p.R) {
              const long long idx = sbase + ((long long)n * p.O + o) * p.L + l;
              if (okind == ATX_OUT_I32) ((int*)p.y)[idx] = v[e];
              else ((float*)p.y)[idx] = f[e];
            }
            if (++l == p.L) { l = 0; ++n; }
          }
        }
      }
    }
  }
}

struct Plan { int wcn, tiles_r, tiles_c, splits, kq; };

// Split count by a cost model in quads of one workgroup: rounds of the
// persistent grid x (quads per split + 6 for a tile's prologue and
// epilogue), plus for S > 1 the partial slices (8 bytes per output per
// split) and the reduce launch.  S is at least ceil(K / KMAX).
static Plan make_plan(int N, int K, int L, int O) {
  Plan pl;
  const long long R = (long long)N * L;
  pl.wcn = O <= 64 ? 1 : 2;
  pl.tiles_r = (int)cdiv(R, 64 * (NWAVE / pl.wcn));
  pl.tiles_c = (int)cdiv(O, 64 * pl.wcn);
  const int nq = (int)cdiv(K, 4);
  const long long tiles = (long long)pl.tiles_r * pl.tiles_c;
  const int smin = (int)cdiv(K, KMAX);
  const double slice = (double)R * O / 2.0e6;     // quads per partial slice round trip
  int best = smin;
  double best_cost = -1.0;
  for (int S = smin; S <= std::max(smin, 32); ++S) {
    const int kq = (int)cdiv(nq, S);
    if (S > smin && kq < 8) break;
    const int splits = (int)cdiv(nq, kq);
    const double cost = (double)cdiv(tiles * splits, 256) * (kq + 6) +
                        (splits > 1 ? 4.0 + splits * slice : 0.0);
    if (best_cost < 0 || cost < best_cost) { best = splits; best_cost = cost; }
  }
  pl.kq = (int)cdiv(nq, best);
  pl.splits = (int)cdiv(nq, pl.kq);
  return pl;
}

}  // namespace ohf
}  // namespace atx

using namespace atx;

extern "C" {

long long atx_lut_gemm_narrow_workspace_bytes(int N, int K, int L, int O) {
  if (N <= 0 || K <= 0 || L <= 0 || O <= 0) return 0;
  const ohf::Plan pl = ohf::make_plan(N, K, L, O);
  return pl.splits > 1 ? (long long)pl.splits * N * O * L * 4 : 0;
}

static int narrow_run(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad, int N, int K,
                      int L, int O, const uint16_t* lut16t, int lut_class, int wbase,
                      atx_gemm_epilogue ep, const U8Terms& u8, void* y, void* workspace,
                      hipStream_t stream);

int atx_lut_gemm_narrow(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad, int N, int K,
                        int L, int O, const uint16_t* lut16t, int lut_class, int wbase,
                        atx_gemm_epilogue ep, void* y, void* workspace, hipStream_t stream) {
  ATX_REQUIRE_EPILOGUE(ep, "atx_lut_gemm_narrow");
  ATX_REQUIRE(ep.out_kind >= ATX_OUT_F32 && ep.out_kind <= ATX_OUT_DEQUANT,
              "atx_lut_gemm_narrow: bad out_kind");
  return narrow_run(xt, Rpad, wt, Opad, N, K, L, O, lut16t, lut_class, wbase, ep, U8Terms{}, y,
                    workspace, stream);
}

int atx_lut_gemm_narrow_uint8(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad, int N,
                              int K, int L, int O, const uint16_t* lut16t, int lut_class,
                              const float* scale_x, const float* scale_w, const float* bias,
                              const float* xsum, const float* wsum, const float* zero_x,
                              const float* zero_w, float* y, void* workspace,
                              hipStream_t stream) {
  ATX_REQUIRE(K > 0, "atx_lut_gemm_narrow_uint8: needs K > 0");
  ATX_REQUIRE((long long)N * L * O == 0 ||
                  (scale_x && scale_w && xsum && wsum && zero_x && zero_w),
              "atx_lut_gemm_narrow_uint8: null pointer");
  const atx_gemm_epilogue ep =
      atx_gemm_epilogue_make(OUT_DEQUANT_U8, scale_x, scale_w, bias, nullptr);
  const U8Terms u8{xsum, wsum, zero_x, zero_w, (float)K};
  return narrow_run(xt, Rpad, wt, Opad, N, K, L, O, lut16t, lut_class, 0, ep, u8, y, workspace,
                    stream);
}

static int narrow_run(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad, int N, int K,
                      int L, int O, const uint16_t* lut16t, int lut_class, int wbase,
                      atx_gemm_epilogue ep, const U8Terms& u8, void* y, void* workspace,
                      hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0 && O >= 0, "atx_lut_gemm_narrow: negative size");
  ATX_REQUIRE(lut_class == ATX_LUT_I16 || lut_class == ATX_LUT_U16,
              "atx_lut_gemm_narrow: needs an integer LUT class (int16 or uint16)");
  ATX_REQUIRE(wbase >= 0 && wbase <= 240, "atx_lut_gemm_narrow: wbase must be in [0, 240]");
  ATX_REQUIRE(ep.out_kind != ATX_OUT_DEQUANT || (ep.scale_x && ep.scale_w),
              "atx_lut_gemm_narrow: dequant epilogue needs scale_x and scale_w");
  const long long R = (long long)N * L;
  if (R * O == 0) return ATX_OK;
  if (K == 0)   // empty contraction: the general kernel runs the epilogue alone
    return atx_lut_gemm(xt, Rpad, wt, Opad, N, K, L, O, lut16t, nullptr, lut_class, ep, y,
                        workspace, stream);
  ATX_REQUIRE(xt && wt && lut16t && y, "atx_lut_gemm_narrow: null pointer");
  ATX_REQUIRE(Rpad >= R && Rpad % ATX_ROW_TILE == 0, "atx_lut_gemm_narrow: bad Rpad %d", Rpad);
  ATX_REQUIRE(Opad >= O && Opad % 32 == 0, "atx_lut_gemm_narrow: bad Opad %d", Opad);
  ATX_REQUIRE((long long)operand_rows(K) * Rpad * 2 < 0x7fffffffLL &&
                  (long long)K * Opad < 0x7fffffffLL,
              "atx_lut_gemm_narrow: operand too large for 32-bit buffer offsets");
  const ohf::Plan pl = ohf::make_plan(N, K, L, O);
  ohf::Params p{};
  p.xt = xt; p.Rpad = Rpad; p.wt = wt; p.Opad = Opad; p.lut16t = lut16t;
  p.K = K; p.R = (int)R; p.L = L; p.O = O; p.wbase = wbase;
  p.is_signed = lut_class == ATX_LUT_I16;
  p.out_kind = ep.out_kind; p.y = y;
  p.sx = ep.scale_x; p.sw = ep.scale_w; p.bias = ep.bias; p.u8 = u8;
  p.tiles_r = pl.tiles_r; p.tiles_c = pl.tiles_c; p.splits = pl.splits; p.kq = pl.kq;
  const long long tiles = (long long)pl.tiles_r * pl.tiles_c * pl.splits;
  ATX_REQUIRE(tiles < 0x7fffffffLL, "atx_lut_gemm_narrow: grid too large");
  p.tiles = (int)tiles;
  p.xt_bytes = (unsigned)((long long)operand_rows(K) * Rpad * 2);
  p.wt_bytes = (unsigned)((long long)K * Opad);
  const long long numel = R * O;
  if (pl.splits > 1) {
    ATX_REQUIRE(workspace, "atx_lut_gemm_narrow: the split plan needs a workspace of %lld bytes",
                (long long)pl.splits * numel * 4);
    p.y = workspace;
    p.split_stride = numel;
  }
  const int blocks = (int)std::min<long long>(256, ((tiles + 7) / 8) * 8);
  int rc = timing_mark(false, stream);
  if (rc != ATX_OK) return rc;
  if (pl.wcn == 1)
    hipLaunchKernelGGL(ohf::onehot_gemm_kernel<1>, dim3(blocks), dim3(ohf::NT), 0, stream, p);
  else
    hipLaunchKernelGGL(ohf::onehot_gemm_kernel<2>, dim3(blocks), dim3(ohf::NT), 0, stream, p);
  rc = check_launch("onehot_gemm_kernel");
  if (rc == ATX_OK) rc = timing_mark(true, stream);
  if (rc != ATX_OK || pl.splits == 1) return rc;
  return launch_split_reduce((const int*)workspace, pl.splits, numel, O, L, ep, y, stream, u8);
}

}  // extern "C"
