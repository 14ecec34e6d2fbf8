// LUT GEMM forward for gfx950: y[n,o,l] = sum_k LUT[xi(n,k,l)][wi(o,k)].
//
// Kernel structure ("expanded tables", four to an LDS line):
//   A workgroup owns a tile of ATX_ROW_TILE (2048) rows r = n*L + l and
//   ATX_COL_TILE (32) output channels.  For every k it builds, in LDS, the
//   table E_k[v][o] = LUT16[v][wi(o,k)] (256 rows x 32 channels x 16 bit =
//   16 KiB) from the transposed 16-bit LUT image (L2-resident, 128 KiB), then
//   every lane looks up E_k[xi(r,k)][o..o+7] for its rows with one 16-byte
//   LDS read and adds the eight 16-bit entries into int32 accumulators
//   (exact).  Table bytes written per lookup are 512 / ATX_ROW_TILE, so the
//   tall, narrow tile halves the table-build cost of a 1024 x 64 tile with
//   the same accumulators per lane.
//
//   LDS bank layout.  gfx950's LDS has 64 banks (256 bytes per clock) and
//   serves a 16-byte read in passes of 16 lanes.  An E row is 64 bytes, so a
//   pass covers four rows, and rows landing in the same quarter of the banks
//   serialize.  Four consecutive tables therefore share each 256-byte LDS
//   line: line v holds row v of table 4j+q in quarter q.  In sub-step s of
//   quad j, row group rg reads table 4j + ((rg + s) & 3); the four row
//   groups of a pass read four different quarters whatever their rows, so
//   the reads are conflict-free (130 TB/s measured, against 66 TB/s for
//   random quarters).  Over the quad's four sub-steps every lane reads all
//   four tables.  Within a quarter, the 16-byte chunk for channels 8g..8g+7
//   of row v sits at position g ^ ((v >> 1) & 3).  The activation operand is
//   pre-encoded as the byte offset v*256 + ((v >> 1) & 3)*16 ("row offset");
//   a lane's address is row_offset ^ (g*16 | quarter*64 | buffer*65536).
//
//   Table build: two quad buffers (128 KiB).  In sub-step s of quad j every
//   wave writes its part of table 4(j+1)+s into the other buffer: wave w
//   covers channel group w % 4 for rows 128(w / 4) .. +127; its eight
//   weight indices are wave-uniform (one vector load read back with
//   v_readlane); lane t loads the dwords LUT16T[w_c][v0, v0+1] (v0 = row
//   pair of the lane) of the eight channels c (buffer loads, scalar offsets),
//   interleaves them with v_perm into the 16-byte chunks of rows v0 and v0+1
//   and stores each with one ds_write_b128.  One barrier per quad (four
//   k-steps) orders the build of quad j+1 and the reads of quad j.
//
//   Threads: 512 (8 waves).  Lane = (row group rg 0..15, channel group g);
//   wave w owns rows 256w .. 256w+255 of the tile and lane (rg, g) the rows
//   64h + 4rg + m (h, m = 0..3) x 8 channels = 128 int32 accumulators
//   (256-VGPR budget at 2 waves per SIMD).  Four consecutive rows per lane
//   let the epilogue store every (channel, h) as one 16-byte vector, and the
//   sixteen row groups of a channel fill two 128-byte lines, so results go
//   from registers straight to HBM with all waves storing at once.
//
// Reference: bgemm_lut_u8_kernel / bgemm_mainloop
// (csrc/claude/bgemm_lut_kernels.cuh:183-387) computes the same sum with a
// 16-bit LUT gathered through L1 and fp32 accumulation.

#include "atx_internal.h"
#include "atx_tiles.h"

#include <algorithm>
#include <mutex>
#include <stdlib.h>
#include <string.h>
#include <type_traits>

namespace atx {

constexpr int RT = ATX_ROW_TILE;   // rows per workgroup (2048)
constexpr int OT = ATX_COL_TILE;   // channels per workgroup (32)
constexpr int CG = OT / 8;         // 16-byte channel chunks per table row (4)
constexpr int NRG = 64 / CG;       // row groups per wave (16)
constexpr int RQ = 4;              // consecutive rows per lane quad
constexpr int NQ = 4;              // quads per lane (stride NRG * RQ rows)
constexpr int RPL = RQ * NQ;       // rows per lane (16)
constexpr int RPW = NRG * RPL;     // rows per wave (256)
constexpr int NWAVE = RT / RPW;    // waves per workgroup (8)
constexpr int NT = 64 * NWAVE;     // threads per workgroup (512)
constexpr int TPL = 4;             // tables per LDS line (quarters)
constexpr int LINE = 256;          // bytes per LDS line
constexpr int QTAB = 256 * LINE;   // one quad of tables (64 KiB)
constexpr int SMEM_BYTES = 2 * QTAB;          // two quad buffers (128 KiB)
static_assert(QTAB == 1 << 16, "quad buffer select is bit 16 of a read address");
static_assert(CG == 4 && NRG == 16 && NWAVE == 8, "tile geometry");
static_assert(TPL * CG * 16 == LINE, "four 64-byte table rows per line");
static_assert(2 * NWAVE == 16 && 256 / 2 == 64 * (NWAVE / CG),
              "a table is 8 waves x 64 lanes x one row pair");

// K limits for exact int32 partial sums (entries up to 32767 / 65535).
constexpr int KMAX_I16 = 65536;
constexpr int KMAX_U16 = 32768;

struct GemmParams {
  const uint16_t* xt; int Rpad;
  const uint8_t* wt; int Opad;
  const uint16_t* lut16t;
  const float* lutf32t;
  int K, R, L, O;
  int k_chunk, splits, tiles_r, tiles_o;
  // Rows per tile: RT, or fewer (a multiple of RPW) when R / RT leaves the
  // last tile mostly empty, so every tile carries about R / tiles_r rows.
  // Waves whose rows lie past the tile (wave * RPW >= rt) build tables but
  // accumulate and store nothing.
  int rt;
  int out_kind;                 // ATX_OUT_*; splits > 1 => raw int32 partials
  void* y;
  long long split_stride;       // elements per partial slice
  const float* sx; const float* sw; const float* bias;
  // Stream-K schedule (sk_per > 0) of G workgroups: workgroup w first runs
  // the whole tiles w, w + G, ... below sk_dp (sk_dp = G * full rounds),
  // then quads [w * sk_per, (w + 1) * sk_per) of the tile-major (tile, quad)
  // space of the remaining tiles, nqt quads per tile; a remaining tile cut by
  // a workgroup boundary adds its int32 sums into slot
  // floor(tail tile * nqt / sk_per) of skws.
  int sk_per, nqt, sk_dp, sk_g;
  int* skws;
  // Device flag (or null): nonzero when every activation index of the rows
  // below R is at least 128 (x >= 0 before an int8 fake-quant).  The tables
  // are then built for rows 128..255 only (upper-half tables).
  const int* x_upper;
};

// ------------------------------------------------------------------ prepare
__global__ void lut_prepare_kernel(const float* __restrict__ lut,
                                   uint16_t* __restrict__ out16t,
                                   float* __restrict__ outf32t,
                                   int* __restrict__ flags) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;   // 65536 entries
  const float v = lut[i];
  const float r = __builtin_rintf(v);
  const bool is_int = (v == r);
  const bool ok16 = is_int && fabsf(v) <= 32767.0f;
  const bool oku16 = is_int && v >= 0.0f && v <= 65535.0f;
  if (!ok16) flags[0] = 1;     // benign race: every writer stores 1
  if (!oku16) flags[1] = 1;
  const unsigned short v16 =
      (ok16 || oku16) ? (unsigned short)(unsigned)(int)r : (unsigned short)0;
  const int t = ((i & 255) << 8) | (i >> 8);             // [x][w] -> [w][x]
  out16t[t] = v16;
  outf32t[t] = v;
}

// ------------------------------------------------------------- operand pack
// xt[slot][r] = row_offset(x[n][operand_tap(slot, r)][l]) for r < R
// (r = n*L + l); 0 for r >= R and taps >= K.  A thread writes the four rows
// of a quad (one tap) as one 8-byte store; when L % 4 == 0 the quad is four
// consecutive elements of one x row, read with one 4- (u8) or 16-byte (fp32)
// load (`vec`: L % 4 == 0 and the pointers aligned for it).  The grid stride over quads is a multiple of 4, so every thread keeps
// one tap per slot.
template <typename T>
__global__ void pack_x_kernel(const T* __restrict__ x, int N, int K, int L,
                              int offset, uint8_t* __restrict__ xq,
                              uint16_t* __restrict__ xt, int Rpad, bool vec,
                              int* __restrict__ upper) {
  const int R = N * L;
  const int q0 = blockIdx.x * blockDim.x + threadIdx.x;
  const int qstride = gridDim.x * blockDim.x;
  const int nquad = Rpad >> 2;
  bool low = false;             // some index of rows < R and taps < K is < 128
  for (int slot = blockIdx.y; slot < operand_rows(K); slot += gridDim.y) {
    const int k = operand_tap(slot, q0 << 2);
    uint16_t* dst = xt + (long long)slot * Rpad;
    for (int q = q0; q < nquad; q += qstride) {
      const int r0 = q << 2;
      unsigned v[4] = {0u, 0u, 0u, 0u};
      bool any = false;
      if (k < K && r0 < R) {
        any = true;
        int n = r0 / L;
        int l = r0 - n * L;
        if (vec) {
          const long long src = ((long long)n * K + k) * L + l;
          if constexpr (sizeof(T) == 4) {
            const float4 f = *(const float4*)(x + src);
            v[0] = quant_index(f.x, offset); v[1] = quant_index(f.y, offset);
            v[2] = quant_index(f.z, offset); v[3] = quant_index(f.w, offset);
            if (xq) *(uchar4*)(xq + src) = make_uchar4(v[0], v[1], v[2], v[3]);
          } else {
            const unsigned w = *(const unsigned*)(x + src);
            v[0] = w & 255u; v[1] = (w >> 8) & 255u; v[2] = (w >> 16) & 255u; v[3] = w >> 24;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (r0 + e < R) {
              const long long src = ((long long)n * K + k) * L + l;
              if constexpr (sizeof(T) == 4) {
                v[e] = quant_index((float)x[src], offset);
                if (xq) xq[src] = (uint8_t)v[e];
              } else {
                v[e] = (unsigned)x[src];
              }
            }
            if (++l == L) { l = 0; ++n; }
          }
        }
      }
      unsigned off[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool live = any && r0 + e < R;
        off[e] = live ? row_offset(v[e]) : 0u;
        low |= live && v[e] < 128u;
      }
      *(uint2*)(dst + r0) = make_uint2(off[0] | (off[1] << 16), off[2] | (off[3] << 16));
    }
  }
  if (upper && low) upper[0] = 0;        // benign race: every writer stores 0
}

// u8 row operand with one quad of rows and one quad of slots per thread
// (blockIdx.y = slot quad): the four taps' bytes of the quad are read
// together (one 4-byte load each when `vec`, as in pack_x_kernel) and
// written as four 8-byte pieces, so every thread moves 16 elements.
__global__ void __launch_bounds__(256)
pack_x_u8_quads_kernel(const uint8_t* __restrict__ x, int N, int K, int L,
                       uint16_t* __restrict__ xt, int Rpad, bool vec, int* __restrict__ upper) {
  const int q = blockIdx.x * 256 + threadIdx.x;
  if (q >= (Rpad >> 2)) return;
  const int R = N * L;
  const int r0 = q << 2;
  long long base[4];
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
  unsigned v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = k4 | ((q + u) & 3);            // this quad's tap of slot k4 + u
    const long long kl = (long long)min(k, K - 1) * L;
    if (vec) {
      v[u] = (k < K && valid) ? *(const unsigned*)(x + base[0] + kl) : 0u;
    } else {
      v[u] = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (k < K && ((valid >> e) & 1u)) v[u] |= (unsigned)x[base[e] + kl] << (8 * e);
    }
  }
  uint16_t* dst = xt + (long long)k4 * Rpad + r0;
  bool low = false;             // some index of rows < R and taps < K is < 128
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = k4 | ((q + u) & 3);
    unsigned off[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool live = k < K && ((valid >> e) & 1u);
      const unsigned idx = (v[u] >> (8 * e)) & 255u;
      off[e] = live ? row_offset(idx) : 0u;
      low |= live && idx < 128u;
    }
    *(uint2*)(dst + (long long)u * Rpad) =
        make_uint2(off[0] | (off[1] << 16), off[2] | (off[3] << 16));
  }
  if (upper && low) upper[0] = 0;        // benign race: every writer stores 0
}

// Strided operands of the plain (torch.mm-layout) LUT GEMM.  Row operand:
// X[r][k] at X + r*sr + k*sk -> xt[slot][r] = row_offset(index), as pack_x
// (quads of rows share a tap); column operand: Y[c][k] at Y + c*sc + k*sk ->
// wt[k][c] = index.  index = clamp(rint(v) + offset, 0, 255) for fp32, the
// byte for uint8; the optional u8 images get q[r*K + k] / q[c*K + k].
template <typename T>
__global__ void pack_rows_strided_kernel(const T* __restrict__ x, int R, int K, long long sr,
                                         long long sk, int offset, uint8_t* __restrict__ xq,
                                         uint16_t* __restrict__ xt, int Rpad,
                                         int* __restrict__ upper) {
  const int q0 = blockIdx.x * blockDim.x + threadIdx.x;
  const int qstride = gridDim.x * blockDim.x;
  const int nquad = Rpad >> 2;
  bool low = false;             // some index of rows < R and taps < K is < 128
  for (int slot = blockIdx.y; slot < operand_rows(K); slot += gridDim.y) {
    const int k = operand_tap(slot, q0 << 2);
    uint16_t* dst = xt + (long long)slot * Rpad;
    for (int q = q0; q < nquad; q += qstride) {
      const int r0 = q << 2;
      unsigned off[4] = {0u, 0u, 0u, 0u};
      if (k < K) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = r0 + e;
          if (r < R) {
            unsigned v;
            if constexpr (sizeof(T) == 4) v = quant_index((float)x[r * sr + k * sk], offset);
            else v = (unsigned)x[r * sr + k * sk];
            if (xq) xq[(long long)r * K + k] = (uint8_t)v;
            off[e] = row_offset(v);
            low |= v < 128u;
          }
        }
      }
      *(uint2*)(dst + r0) = make_uint2(off[0] | (off[1] << 16), off[2] | (off[3] << 16));
    }
  }
  if (upper && low) upper[0] = 0;        // benign race: every writer stores 0
}

template <typename T>
__global__ void pack_cols_strided_kernel(const T* __restrict__ y, int C, int K, long long sc,
                                         long long sk, int offset, uint8_t* __restrict__ yq,
                                         uint8_t* __restrict__ wt, int Opad) {
  const long long total = (long long)K * Opad;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const int k = (int)(i / Opad);
    const int c = (int)(i - (long long)k * Opad);
    unsigned v = 0;
    if (c < C) {
      if constexpr (sizeof(T) == 4) v = quant_index((float)y[c * sc + k * sk], offset);
      else v = (unsigned)y[c * sc + k * sk];
      if (yq) yq[(long long)c * K + k] = (uint8_t)v;
    }
    wt[i] = (uint8_t)v;
  }
}

template <typename T>
__global__ void pack_w_kernel(const T* __restrict__ w, int O, int K, int offset,
                              uint8_t* __restrict__ wq, uint8_t* __restrict__ wt,
                              int Opad) {
  const long long total = (long long)K * Opad;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const int k = (int)(i / Opad);
    const int o = (int)(i - (long long)k * Opad);
    unsigned v = 0;
    if (o < O) {
      const long long src = (long long)o * K + k;
      if constexpr (sizeof(T) == 4) {
        v = quant_index((float)w[src], offset);
        if (wq) wq[src] = (uint8_t)v;
      } else {
        v = (unsigned)w[src];
      }
    }
    if (wt) wt[i] = (uint8_t)v;
  }
}

// ------------------------------------------------------------- main kernel
// Accumulates one 16-byte table chunk (channels 2m, 2m+1 in dword m, the
// even channel in the low half) into a row's pair accumulators:
// a[2m] += d_m, the whole dword, and a[2m+1] += d_m >> 16, the high entry
// (sign-extended for signed tables).  The even channels' sums are recovered
// once per tile segment (pair_sums): a[2m] - (a[2m+1] << 16), less the bias
// of the low entries for signed tables.  One add of each pair is a plain
// 32-bit VOP2 add, which gfx950 issues at about 1.7x the rate of the SDWA
// form that extracts a 16-bit half.
template <bool SIGNED>
__device__ __forceinline__ void add8(int (&a)[8], const uint4 e) {
  const unsigned d[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[2 * i] = (int)((unsigned)a[2 * i] + d[i]);
    if constexpr (SIGNED) a[2 * i + 1] += ((int)d[i]) >> 16;
    else a[2 * i + 1] += (int)(d[i] >> 16);
  }
}

// Signed tables store their low (even-channel) entries biased by 2^15, so
// that a dword's value is exactly hi * 2^16 + (lo + 2^15) with the low part
// in [0, 2^16): summed over T tables, the even channel's sum is
// S - (H << 16) - 2^15 T (mod 2^32; exact within the int32 bound).
constexpr unsigned LOW_BIAS = 0x8000u;

// Turns the pair accumulators of the lane's rows into channel sums after
// `tables` tables (every table accumulated, all-zero ones included: their
// biased low entries are exactly LOW_BIAS).
template <bool SIGNED>
__device__ __forceinline__ void pair_sums(int (&acc)[RPL][8], int tables) {
  const unsigned bias = SIGNED ? LOW_BIAS * (unsigned)tables : 0u;
#pragma unroll
  for (int j = 0; j < RPL; ++j)
#pragma unroll
    for (int m = 0; m < 4; ++m)
      acc[j][2 * m] =
          (int)((unsigned)acc[j][2 * m] - ((unsigned)acc[j][2 * m + 1] << 16) - bias);
}

// Table-build registers: the LUT16T dwords (entries v0, v0+1) of the wave's
// eight channels.
struct Rows { unsigned d[8]; };
// Eight weight indices (channels o0 + 8*og .. +7) at k, wcol = &wt[k][o0 +
// 8*og].  Lane parity picks the dword (indices 0-3 / 4-7) so the load is a
// vector load: a scalar load would share the LDS wait counter and,
// completing out of order, force every LDS wait of the step to drain it.
__device__ __forceinline__ unsigned load_w8(const uint8_t* wcol, int lane) {
  return __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(wcol, 8), (lane & 1) * 4, 0, 0);
}

// Dword at entries (v0, v0+1) of LUT16T row w_c for every channel c of the
// group, v0 = 2*lane + sbase/2.  Row offsets are wave-uniform (read from
// lanes 0 and 1 of the weight-index register).
__device__ __forceinline__ void load_rows(Rows& r, __amdgpu_buffer_rsrc_t lut, unsigned wv,
                                          int lane, int sbase) {
  const unsigned w_lo = __builtin_amdgcn_readlane(wv, 0);
  const unsigned w_hi = __builtin_amdgcn_readlane(wv, 1);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const unsigned wc = ((c < 4 ? w_lo : w_hi) >> (8 * (c & 3))) & 255u;
    r.d[c] = __builtin_amdgcn_raw_buffer_load_b32(lut, lane * 4, (int)(wc * 512u) + sbase, 0);
  }
}

// Writes the lane's two 16-byte chunks (rows v0 and v0+1, channels
// 8*og .. 8*og+7) at smem + wb (row v0's chunk; row v0+1 is one line on).
// Signed tables get their even channels' entries biased (LOW_BIAS).
template <bool SIGNED>
__device__ __forceinline__ void write_table(unsigned char* smem, const Rows& r, int wb) {
  unsigned d[8];
#pragma unroll
  for (int c = 0; c < 8; ++c)
    d[c] = (SIGNED && (c & 1) == 0) ? r.d[c] ^ (LOW_BIAS | (LOW_BIAS << 16)) : r.d[c];
  uint4 lo, hi;      // channel pairs (2m, 2m+1) at v0 (low halves) / v0+1 (high)
  lo.x = __builtin_amdgcn_perm(d[1], d[0], 0x05040100u);
  lo.y = __builtin_amdgcn_perm(d[3], d[2], 0x05040100u);
  lo.z = __builtin_amdgcn_perm(d[5], d[4], 0x05040100u);
  lo.w = __builtin_amdgcn_perm(d[7], d[6], 0x05040100u);
  hi.x = __builtin_amdgcn_perm(d[1], d[0], 0x07060302u);
  hi.y = __builtin_amdgcn_perm(d[3], d[2], 0x07060302u);
  hi.z = __builtin_amdgcn_perm(d[5], d[4], 0x07060302u);
  hi.w = __builtin_amdgcn_perm(d[7], d[6], 0x07060302u);
  *(uint4*)(smem + wb) = lo;
  *(uint4*)(smem + wb + LINE) = hi;
}

// Accumulates one table for this lane's RPL rows.  x holds the rows'
// offsets (two per dword, below 65536); gx XORs in the lane's channel chunk
// (bits 4-5), the table's quarter (bits 6-7) and the quad buffer (bit 16).
// All sixteen reads are issued before the first add, so the lane has a whole
// table step of reads in flight (2.5% faster than two batches of eight).
template <bool SIGNED>
__device__ __forceinline__ void use_table(int (&acc)[RPL][8], const unsigned char* smem,
                                          const XRows& x, unsigned gx) {
  uint4 e[RPL];
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    e[RQ * h] = *(const uint4*)(smem + ((x.v[h].x & 0xffffu) ^ gx));
    e[RQ * h + 1] = *(const uint4*)(smem + ((x.v[h].x >> 16) ^ gx));
    e[RQ * h + 2] = *(const uint4*)(smem + ((x.v[h].y & 0xffffu) ^ gx));
    e[RQ * h + 3] = *(const uint4*)(smem + ((x.v[h].y >> 16) ^ gx));
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) add8<SIGNED>(acc[j], e[j]);
}

// Stores W consecutive results v[0..W-1] of channel o at y[yi..yi+W-1] as
// int32 (kind ATX_OUT_I32, also the split-K partials), fp32, or dequantized
// fp32 (sx * sw[o] * v [+ bias[o]]).
template <int KIND, int W>
__device__ __forceinline__ void put_rows(const GemmParams& p, void* y, long long yi,
                                         int o, const int* v) {
  if constexpr (KIND == ATX_OUT_I32) {
    if constexpr (W == 4) *(int4*)((int*)y + yi) = make_int4(v[0], v[1], v[2], v[3]);
    else ((int*)y)[yi] = v[0];
  } else {
    float f[W];
    if constexpr (KIND == ATX_OUT_F32) {
#pragma unroll
      for (int m = 0; m < W; ++m) f[m] = (float)v[m];
    } else {
      const float sc = p.sx[0] * p.sw[o];
#pragma unroll
      for (int m = 0; m < W; ++m) {
        const float t = (float)v[m] * sc;
        f[m] = p.bias ? p.bias[o] + t : t;
      }
    }
    if constexpr (W == 4) *(float4*)((float*)y + yi) = make_float4(f[0], f[1], f[2], f[3]);
    else ((float*)y)[yi] = f[0];
  }
}

// Writes the lane's accumulators: channel o0 + e, rows r + NRG*RQ*h + m of
// quad h (r = first row of quad 0).  Rows beyond R and channels beyond O are
// dropped.  With L % 4 == 0 a quad never straddles two images and is one
// 16-byte store (r is a multiple of 4); otherwise rows are stored one by one,
// stepping (n, l) across image boundaries.
template <int KIND>
__device__ __forceinline__ void store_tile(const GemmParams& p, void* y,
                                           const int (&acc)[RPL][8], int r, int o0) {
  const bool vec = (p.L & 3) == 0;
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    const int rq = r + NRG * RQ * h;
    if (rq >= p.R) break;
    const int n = rq / p.L;
    const int l = rq - n * p.L;
    if (vec) {
      const long long ybase = (long long)n * p.O * p.L + l;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int o = o0 + e;
        if (o >= p.O) break;
        const int v[RQ] = {acc[RQ * h][e], acc[RQ * h + 1][e], acc[RQ * h + 2][e],
                           acc[RQ * h + 3][e]};
        put_rows<KIND, RQ>(p, y, ybase + (long long)o * p.L, o, v);
      }
    } else {
      int nm = n, lm = l;
#pragma unroll
      for (int m = 0; m < RQ; ++m) {
        if (rq + m >= p.R) break;
        const long long ybase = (long long)nm * p.O * p.L + lm;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int o = o0 + e;
          if (o >= p.O) break;
          put_rows<KIND, 1>(p, y, ybase + (long long)o * p.L, o, &acc[RQ * h + m][e]);
        }
        if (++lm == p.L) { lm = 0; ++nm; }
      }
    }
  }
}

// Sums of one tile segment: rows tile tr, channels tile to, k in [kb, ke).
template <bool SIGNED, bool UPPER>
__device__ __forceinline__ void lut_tile(const GemmParams& p, unsigned char* smem, int tr,
                                         int to, int kb, int ke, int (&acc)[RPL][8]) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane / CG, g = lane % CG;
  const int o0 = to * OT;

  // Table build: wave w writes channel group og = w % 4 for rows
  // 128 hw .. 128 hw + 127 (hw = w / 4); lane t the row pair v0 = 128 hw + 2t,
  // v0 + 1, whose chunk og sits at position og ^ ((v0 >> 1) & 3) =
  // og ^ (t & 3) of quarter q.  wb0 addresses row v0's chunk in quad
  // buffer 0 (buffer 1 is QTAB on); the quarter is an immediate offset
  // (q * 64).
  //
  // UPPER (every activation index >= 128): tables hold rows 128..255 only.
  // They are built in pairs, wave w writing rows 128..255 of channel group og
  // of table 2i + hw: in an even sub-step every wave loads the weight indices
  // of the next pair and writes its table of the current pair, in an odd one
  // it loads the LUT rows of the next pair and writes nothing, so each wave
  // does half the table work of full tables.  Row 0 (the operand's padding
  // rows and taps point there) is set once per kernel to a zero entry.
  const int og = __builtin_amdgcn_readfirstlane(wave % CG);
  const int hw = __builtin_amdgcn_readfirstlane(wave / CG);
  const int vbase = UPPER ? 128 : 128 * hw;             // first table row of the lane pairs
  const int tsel = UPPER ? hw : 0;                      // the wave's table of a pair
  const int sbase = 2 * vbase;                          // its byte offset in a LUT16T row
  const int wb0 = (vbase + 2 * lane) * LINE + ((og ^ (lane & 3)) << 4);
  // Read XOR masks: sub-step s of a quad reads quarter (rg + s) & 3.
  const unsigned gbase = (unsigned)((rg << 6) | (g << 4));

  const int xoff = (wave * RPW + rg * RQ) * 2;          // lane's first quad, bytes
  const uint16_t* __restrict__ xtile = p.xt + (long long)tr * p.rt;
  // wave-uniform: does this wave own rows of the tile?
  const bool active = __builtin_amdgcn_readfirstlane(wave) * RPW < p.rt;
  const uint8_t* __restrict__ wcol = p.wt + o0 + og * 8;
  const __amdgpu_buffer_rsrc_t lutr = buffer_rsrc(p.lut16t, 256 * 256 * 2);
  // Zero-length view of the image: its loads are out of range and return 0,
  // which builds an all-zero table for the steps past the chunk's end.
  const __amdgpu_buffer_rsrc_t lutz = buffer_rsrc(p.lut16t, 0);

#pragma unroll
  for (int j = 0; j < RPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0;

  if (kb < ke) {
    // Sub-steps sigma = 4j + s (tables counted from kb; n of them).  Sub-step
    // sigma issues the loads for the row offsets of sub-step sigma+1, the
    // LUT rows of table sigma+5 and the weight indices of table sigma+6,
    // accumulates from the lane's table of sub-step sigma and writes table
    // sigma+4 (rows loaded one sub-step earlier).  Tables at or past n are
    // built all-zero from lutz; row offsets past the chunk load as 0 (row 0
    // of such a table), so whole quads run without branches.  Scheduling
    // fences keep the loads ahead of the accumulation and the table write
    // (which waits for its LUT rows) behind it.
    const int n = ke - kb;
    const int nq = (n + TPL - 1) / TPL;
    const int slot_bytes = p.Rpad * 2;                  // one k-row of the operand
    // The operand's quads are rotated (slot s of row r holds tap
    // 4j + (((r >> 2) + s) & 3)), so at sub-step s every lane reads slot s:
    // a scalar offset.  Quads past the chunk, and every quad of a wave past
    // the tile (whose rows can lie past the operand's padded rows when a
    // short last tile ends near Rpad), read through an empty view (0).
    auto quad_rows = [&](int j) {                       // descriptor of quad j's slots
      return buffer_rsrc(xtile + (long long)(kb + TPL * j) * p.Rpad,
                         j < nq && active ? TPL * slot_bytes : 0);
    };
    auto wtab = [&](int t) {                            // weight column of table t
      return wcol + (long long)(kb + min(t, n - 1)) * p.Opad;
    };

    XRows xa, xb;
    Rows rows;
    unsigned wnext = 0;                                 // indices of table sigma+5 (UPPER:
                                                        // of the wave's table of the next pair)
    {
      Rows r4;
      if constexpr (UPPER) {
#pragma unroll
        for (int q = 0; q < TPL; q += 2) {
          load_rows(r4, q + tsel < n ? lutr : lutz, load_w8(wtab(q + tsel), lane), lane, sbase);
          write_table<SIGNED>(smem + (q + tsel) * 64, r4, wb0);  // quad 0 -> buffer 0
        }
      } else {
#pragma unroll
        for (int q = 0; q < TPL; ++q) {
          load_rows(r4, q < n ? lutr : lutz, load_w8(wtab(q), lane), lane, sbase);
          write_table<SIGNED>(smem + q * 64, r4, wb0);  // quad 0 -> buffer 0
        }
      }
      load_rows(rows, TPL + tsel < n ? lutr : lutz, load_w8(wtab(TPL + tsel), lane), lane,
                sbase);
      if constexpr (!UPPER) wnext = load_w8(wtab(TPL + 1), lane);
      load_x(xa, quad_rows(0), xoff, 0);
    }
    __syncthreads();

    // One sub-step; B = quad buffer of quad j, S = sub-step within the quad.
    auto sub = [&](auto bc, auto sc, int j, XRows& xcur, XRows& xnext)
        __attribute__((always_inline)) {
      constexpr int B = decltype(bc)::value;
      constexpr int S = decltype(sc)::value;
      const int sigma = TPL * j + S;
      // Issue order = order of use in the next sub-step (the counter of
      // outstanding loads is waited on in order): weight indices (first, to
      // address the LUT rows), row offsets (the accumulation), LUT rows
      // (the table write at the end).  UPPER: even sub-steps load the
      // indices of the pair (sigma+6, sigma+7) and write table sigma+4+hw,
      // odd ones load the LUT rows of table sigma+5+hw.
      constexpr bool kIdx = !UPPER || (S & 1) == 0;     // loads weight indices
      constexpr bool kRows = !UPPER || (S & 1) == 1;    // loads LUT rows
      unsigned wn = wnext;
      if constexpr (kIdx) wn = load_w8(wtab(sigma + 6 + tsel), lane);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (S + 1 < TPL) load_x(xnext, quad_rows(j), xoff, (S + 1) * slot_bytes);
      else load_x(xnext, quad_rows(j + 1), xoff, 0);
      __builtin_amdgcn_sched_barrier(0);
      Rows rn;
      if constexpr (kRows)
        load_rows(rn, sigma + 5 + tsel < n ? lutr : lutz, wnext, lane, sbase);
      __builtin_amdgcn_sched_barrier(0);
      if (active) {
        use_table<SIGNED>(acc, smem, xcur, quarter_mask<S, B>(gbase));
        // Pin the adds here: left free, the compiler sinks them into later
        // steps, past the table write that waits for this step's loads.
#pragma unroll
        for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
          for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(acc[jj][e]));
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kIdx)                               // table sigma+4 (+hw), other buffer
        write_table<SIGNED>(smem + (S + tsel) * 64 + (B ? 0 : QTAB), rows, wb0);
      if constexpr (kRows) rows = rn;
      wnext = wn;
      if constexpr (S == TPL - 1) __syncthreads();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    for (int j = 0; j < nq; j += 2) {
      sub(I0{}, I0{}, j, xa, xb);
      sub(I0{}, I1{}, j, xb, xa);
      sub(I0{}, I2{}, j, xa, xb);
      sub(I0{}, I3{}, j, xb, xa);
      if (j + 1 >= nq) break;
      sub(I1{}, I0{}, j + 1, xa, xb);
      sub(I1{}, I1{}, j + 1, xb, xa);
      sub(I1{}, I2{}, j + 1, xa, xb);
      sub(I1{}, I3{}, j + 1, xb, xa);
    }
    pair_sums<SIGNED>(acc, TPL * nq);
  }
}

// Slot layout of a cut tile (stream-K): value (h, m, e) of thread tid at
// ((RQ * h + m) * 8 + e) * NT + tid, so each atomic of a wave covers 256
// contiguous bytes.
__device__ __forceinline__ long long sk_index(int j, int e, int tid) {
  return (long long)(j * 8 + e) * NT + tid;
}

// Slot of stream-K boundary b (quad position (b + 1) * per), or -1 when that
// boundary does not open a cut tile: the tile containing it must start at or
// after boundary b's predecessor (its first boundary is this one).
// Returns the tail tile index (0-based among the remaining tiles).
__device__ __forceinline__ int sk_slot_tile(const GemmParams& p, int b, long long total) {
  const long long B = (long long)(b + 1) * p.sk_per;
  if (B >= total || B % p.nqt == 0) return -1;
  const long long t = B / p.nqt;
  return (t * p.nqt) / p.sk_per == b ? (int)t : -1;
}

template <bool SIGNED>
__global__ void __launch_bounds__(NT, 1)
lut_gemm_kernel(const GemmParams p) {
  __shared__ __align__(16) unsigned char smem[SMEM_BYTES];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane / CG, g = lane % CG;
  const int lb = logical_block();
  int acc[RPL][8];
  const bool has_rows = wave * RPW < p.rt;   // the wave's rows lie in the tile
  const bool upper = p.x_upper && __builtin_amdgcn_readfirstlane(*p.x_upper) != 0;
  if (upper && tid < 2 * (LINE / 16)) {      // row 0 (line 0) of both quad buffers
    // a zero entry as the table build stores it: signed tables hold their
    // even channels biased by LOW_BIAS, which pair_sums takes off per table
    const unsigned z = SIGNED ? LOW_BIAS : 0u;
    const int c = tid % (LINE / 16);
    *(uint4*)(smem + (tid < LINE / 16 ? 0 : QTAB) + 16 * c) = make_uint4(z, z, z, z);
  }

  if (p.sk_per == 0) {
    int l = lb;
    const int to = l % p.tiles_o; l /= p.tiles_o;
    const int tr = l % p.tiles_r;
    const int s = l / p.tiles_r;
    const int kb = s * p.k_chunk;
    if (upper) lut_tile<SIGNED, true>(p, smem, tr, to, kb, min(p.K, kb + p.k_chunk), acc);
    else lut_tile<SIGNED, false>(p, smem, tr, to, kb, min(p.K, kb + p.k_chunk), acc);
    // ---- epilogue: registers -> HBM, every wave at once (no LDS staging).
    const int r0 = tr * p.rt + wave * RPW + rg * RQ;     // this lane's first quad
    const int oc = to * OT + g * 8;
    if (!has_rows) return;
    if (p.splits > 1)
      store_tile<ATX_OUT_I32>(p, (int*)p.y + (long long)s * p.split_stride, acc, r0, oc);
    else if (p.out_kind == ATX_OUT_I32)
      store_tile<ATX_OUT_I32>(p, p.y, acc, r0, oc);
    else if (p.out_kind == ATX_OUT_F32)
      store_tile<ATX_OUT_F32>(p, p.y, acc, r0, oc);
    else
      store_tile<ATX_OUT_DEQUANT>(p, p.y, acc, r0, oc);
    return;
  }

  // Whole tiles first (the full rounds), then this workgroup's run of the
  // remaining tiles' quads, tile segment by tile segment.
  for (int tile = lb; tile < p.sk_dp; tile += p.sk_g) {
    const int to = tile % p.tiles_o, tr = tile / p.tiles_o;
    __syncthreads();                         // the previous segment's tables are read
    if (upper) lut_tile<SIGNED, true>(p, smem, tr, to, 0, p.K, acc);
    else lut_tile<SIGNED, false>(p, smem, tr, to, 0, p.K, acc);
    const int r0 = tr * p.rt + wave * RPW + rg * RQ;
    const int oc = to * OT + g * 8;
    if (!has_rows) continue;
    if (p.out_kind == ATX_OUT_I32) store_tile<ATX_OUT_I32>(p, p.y, acc, r0, oc);
    else if (p.out_kind == ATX_OUT_F32) store_tile<ATX_OUT_F32>(p, p.y, acc, r0, oc);
    else store_tile<ATX_OUT_DEQUANT>(p, p.y, acc, r0, oc);
  }
  const long long total = ((long long)p.tiles_r * p.tiles_o - p.sk_dp) * p.nqt;
  long long it = (long long)lb * p.sk_per;
  const long long end = min(total, it + p.sk_per);
  while (it < end) {
    const int tt = (int)(it / p.nqt);        // tail tile
    const int q0 = (int)(it - (long long)tt * p.nqt);
    const int q1 = (int)min((long long)p.nqt, q0 + (end - it));
    const int tile = p.sk_dp + tt;
    const int to = tile % p.tiles_o, tr = tile / p.tiles_o;
    __syncthreads();                         // the previous segment's tables are read
    if (upper) lut_tile<SIGNED, true>(p, smem, tr, to, TPL * q0, min(p.K, TPL * q1), acc);
    else lut_tile<SIGNED, false>(p, smem, tr, to, TPL * q0, min(p.K, TPL * q1), acc);
    if (!has_rows) {
      // nothing to store or add (the slots' rows of this wave stay zero)
    } else if (q0 == 0 && q1 == p.nqt) {
      const int r0 = tr * p.rt + wave * RPW + rg * RQ;
      const int oc = to * OT + g * 8;
      if (p.out_kind == ATX_OUT_I32) store_tile<ATX_OUT_I32>(p, p.y, acc, r0, oc);
      else if (p.out_kind == ATX_OUT_F32) store_tile<ATX_OUT_F32>(p, p.y, acc, r0, oc);
      else store_tile<ATX_OUT_DEQUANT>(p, p.y, acc, r0, oc);
    } else {
      int* slot = p.skws + (((long long)tt * p.nqt) / p.sk_per) * (long long)(RPL * 8 * NT);
#pragma unroll
      for (int j = 0; j < RPL; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          __hip_atomic_fetch_add(slot + sk_index(j, e, tid), acc[j][e], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    }
    it += q1 - q0;
  }
}

// Zeroes the slots of the cut tiles (block b = slot b).
__global__ void __launch_bounds__(NT)
sk_clear_kernel(const GemmParams p) {
  const long long total = ((long long)p.tiles_r * p.tiles_o - p.sk_dp) * p.nqt;
  if (sk_slot_tile(p, blockIdx.x, total) < 0) return;
  int* slot = p.skws + (long long)blockIdx.x * (RPL * 8 * NT);
  for (int j = 0; j < RPL * 8; ++j) slot[(long long)j * NT + threadIdx.x] = 0;
}

// Epilogue of the cut tiles: each thread reloads the sums it would have held
// and stores them as the main kernel does.
__global__ void __launch_bounds__(NT)
sk_finish_kernel(const GemmParams p) {
  const long long total = ((long long)p.tiles_r * p.tiles_o - p.sk_dp) * p.nqt;
  const int tt = sk_slot_tile(p, blockIdx.x, total);
  if (tt < 0) return;
  const int tile = p.sk_dp + tt;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane / CG, g = lane % CG;
  const int* slot = p.skws + (long long)blockIdx.x * (RPL * 8 * NT);
  int acc[RPL][8];
#pragma unroll
  for (int j = 0; j < RPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = slot[sk_index(j, e, tid)];
  const int to = tile % p.tiles_o, tr = tile / p.tiles_o;
  const int r0 = tr * p.rt + wave * RPW + rg * RQ;
  const int oc = to * OT + g * 8;
  if (wave * RPW >= p.rt) return;            // rows past the tile
  if (p.out_kind == ATX_OUT_I32) store_tile<ATX_OUT_I32>(p, p.y, acc, r0, oc);
  else if (p.out_kind == ATX_OUT_F32) store_tile<ATX_OUT_F32>(p, p.y, acc, r0, oc);
  else store_tile<ATX_OUT_DEQUANT>(p, p.y, acc, r0, oc);
}

// Split-K reduction: exact int64 sum of int32 partials, then the epilogue.
// One output per thread (any size / alignment).
__global__ void split_reduce1_kernel(const int* __restrict__ ws, int S,
                                     long long numel, int O, int L, int out_kind,
                                     void* __restrict__ y, const float* sx,
                                     const float* sw, const float* bias, U8Terms u8) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < numel;
       i += (long long)gridDim.x * blockDim.x) {
    long long a = 0;
    for (int s = 0; s < S; ++s) a += ws[(long long)s * numel + i];
    if (out_kind == ATX_OUT_I32) {
      ((int*)y)[i] = (int)a;
    } else if (out_kind == ATX_OUT_F32) {
      ((float*)y)[i] = (float)a;
    } else if (out_kind == OUT_DEQUANT_U8) {
      const long long nl = i / L;              // n * O + o
      const int o = (int)(nl % O), l = (int)(i - nl * L);
      const long long n = nl / O;
      const float z = u8.zx[0], zo = u8.zw[o];
      ((float*)y)[i] = u8_dequant((float)a, u8.xs[n * L + l], zo, z * u8.ws[o],
                                  (u8.K * z) * zo, sx[0] * sw[o], bias, bias ? bias[o] : 0.f);
    } else {
      const int o = (int)((i / L) % O);
      const float sc = sx[0] * sw[o];
      const float t = (float)a * sc;
      ((float*)y)[i] = bias ? bias[o] + t : t;
    }
  }
}

// Four consecutive outputs per thread (16-byte partial loads); numel % 4 == 0.
__global__ void split_reduce_kernel(const int* __restrict__ ws, int S,
                                    long long numel, int O, int L, int out_kind,
                                    void* __restrict__ y, const float* sx,
                                    const float* sw, const float* bias, U8Terms u8) {
  for (long long q = blockIdx.x * (long long)blockDim.x + threadIdx.x; q < (numel >> 2);
       q += (long long)gridDim.x * blockDim.x) {
    const long long i = q << 2;
    long long a[4] = {0, 0, 0, 0};
    for (int s = 0; s < S; ++s) {
      const int4 v = *(const int4*)(ws + (long long)s * numel + i);
      a[0] += v.x; a[1] += v.y; a[2] += v.z; a[3] += v.w;
    }
    if (out_kind == ATX_OUT_I32) {
      *(int4*)((int*)y + i) = make_int4((int)a[0], (int)a[1], (int)a[2], (int)a[3]);
    } else if (out_kind == ATX_OUT_F32) {
      *(float4*)((float*)y + i) =
          make_float4((float)a[0], (float)a[1], (float)a[2], (float)a[3]);
    } else if (out_kind == OUT_DEQUANT_U8) {
      long long nl = i / L;                    // n * O + o
      int l = (int)(i - nl * L), o = (int)(nl % O);
      long long n = nl / O;
      const float z = u8.zx[0], kz = u8.K * z, s0 = sx[0];
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float zo = u8.zw[o];
        f[e] = u8_dequant((float)a[e], u8.xs[n * L + l], zo, z * u8.ws[o], kz * zo,
                          s0 * sw[o], bias, bias ? bias[o] : 0.f);
        if (++l == L) { l = 0; if (++o == O) { o = 0; ++n; } }
      }
      *(float4*)((float*)y + i) = make_float4(f[0], f[1], f[2], f[3]);
    } else {
      long long nl = i / L;                    // n * O + o
      int l = (int)(i - nl * L), o = (int)(nl % O);
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float sc = sx[0] * sw[o];
        const float t = (float)a[e] * sc;
        f[e] = bias ? bias[o] + t : t;
        if (++l == L) { l = 0; if (++o == O) o = 0; }
      }
      *(float4*)((float*)y + i) = make_float4(f[0], f[1], f[2], f[3]);
    }
  }
}

// Split plan shared by the workspace query and the launch.  sk_per > 0
// selects the stream-K schedule (PLAN_CUS workgroups, sk_per quads each).
struct Plan { int tiles_r, tiles_o, splits, k_chunk, sk_per, nqt, sk_dp, rt; };

// Compute units of a full MI355X (one resident workgroup each: the kernel's
// 8 waves hold 2 waves per SIMD at its register budget).  A constant, not a
// device query, so the workspace query and the launch always agree.
constexpr int PLAN_CUS = 256;

// Plan by a cost model in units of one k-step of one full-tile workgroup,
// over the rows per tile rt (2048, 1792, 1536, 1280 or 768, keeping
// ceil(R / rt) tiles inside the operand's padded rows) and the split-K count S:
//   ceil(tiles(rt) * S / CUs) rounds x (k-chunk + 6 fixed steps) x f(rt)
//   + for S > 1: 4 steps for the reduce launch and S x (R*O / 600000) steps
//     for writing and re-reading one int32 partial slice,
// with f(rt) = 0.7 + 0.3 rt / 2048 the cost of a k-step of a smaller tile (the
// table build, its loads and the quad barrier do not shrink with the rows).
// Fitted to a sweep of (rt, S) over the 19 distinct ResNet-50 layer shapes
// at batch 64 (the model's picks land within 0.2% of the sweep's best);
// rt = 1024 is left out (slower than 768 or 1280 on every shape measured).
// k-chunks are whole quads of tables (multiples of 4); S is at least
// ceil(K / kmax), the exact-int32 bound of one pass, and the smallest cost
// wins (ties: the larger rt, then the smaller S).
// Stream-K (K <= kmax, at the default rt): floor(tiles / CUs) full rounds of
// whole tiles, then the T = tail tiles * ceil(K/4) quads of the rest dealt
// out evenly, per = ceil(T / CUs) quads per workgroup, which ends the
// partial last round.  Cost, fitted to the split-K / stream-K times of the
// 19 distinct ResNet-50 layer shapes at batch 64 (~0.95 us per k-step):
//   rounds * (K + 14) + 4 * per + 14 per tail segment a workgroup runs
//   (ceil(per / nqt) + 1 at most; table prologue and atomic sums) + 0.1 per
//   cut tile (its 256 KiB slot) + 45 for the clear / finish launches.
// It is taken when cheaper than the best split-K plan (5 of the 19 shapes,
// e.g. K = 576 at 56 x 56 with 64 channels: 460 against 491 us).  With the
// upper-half tables (x_upper given: `upper`) a k-step costs ~0.74 us instead
// of ~0.95 while the cuts' atomics, clears and finishes do not shrink; refit
// on the four stream-K shapes of the 52 ResNet-50 layers at batch 64, a cut
// costs ~0.7 k-steps there (0.1 with full tables), which hands K = 576 at
// 56 x 56 with 64 channels (513 -> 467 us) and K = 512 at 28 x 28 with 256
// (461 -> 420 us) to split-K.
// ATX_LUT_SCHEDULE (environment: auto | split | stream_k) overrides the
// choice; ATX_LUT_ROWS and ATX_LUT_SPLITS force the rows per tile and the
// split count (split-K plans), for measurement.
// ws_limit >= 0 caps the workspace: split counts whose int32 partials exceed
// it are not considered; when even the smallest admissible split count (set
// by the int32-exactness bound) needs more, the plan's splits is -1.
constexpr long long SK_SLOT_BYTES = (long long)(PLAN_CUS - 1) * RT * OT * 4;

static Plan make_plan(int N, int K, int L, int O, int kmax, long long ws_limit = -1,
                      bool upper = false) {
  Plan pl;
  const long long R = (long long)N * L;
  pl.tiles_r = (int)cdiv(R, RT);
  // the fewest whole waves of rows that cover R in tiles_r tiles
  pl.rt = R > 0 ? (int)std::min<long long>(RT, cdiv(cdiv(R, pl.tiles_r), RPW) * RPW) : RT;
  pl.tiles_o = (int)cdiv(O, OT);
  pl.sk_per = 0;
  pl.sk_dp = 0;
  pl.nqt = (int)cdiv(K, TPL);
  if (K <= 0) { pl.splits = 1; pl.k_chunk = 1; return pl; }
  const char* sched = getenv("ATX_LUT_SCHEDULE");
  const bool force_sk = sched && !strcmp(sched, "stream_k");
  const char* force_rows = getenv("ATX_LUT_ROWS");
  const char* force_s = getenv("ATX_LUT_SPLITS");
  const long long cus = PLAN_CUS;
  const int smin = (int)cdiv(K, kmax);
  const int fs = force_s ? std::max(smin, atoi(force_s)) : 0;
  const double slice = (double)R * O / 600000.0;
  const long long rows_cap = cdiv(R, RT) * RT;
  static const int kRows[] = {2048, 1792, 1536, 1280, 768};
  int cand[6], nc = 0;
  if (force_rows) {
    const int rt = atoi(force_rows);
    if (rt >= RPW && rt <= RT && rt % RPW == 0 && R > 0 && cdiv(R, rt) * rt <= rows_cap)
      cand[nc++] = rt;
  }
  if (nc == 0) {
    if (force_sk || R <= 0) {
      cand[nc++] = pl.rt;
    } else {
      cand[nc++] = pl.rt;
      for (int rt : kRows)
        if (rt < pl.rt && cdiv(R, rt) * rt <= rows_cap) cand[nc++] = rt;
    }
  }
  long long best_kc = cdiv(cdiv(K, smin), TPL) * TPL;
  int best_rt = pl.rt;
  double best_cost = 0.0;
  bool found = false;
  for (int c = 0; c < nc; ++c) {
    const int rt = cand[c];
    const long long tiles = cdiv(R, rt) * pl.tiles_o;
    const double f = 0.7 + 0.3 * rt / RT;
    for (int S = fs ? fs : smin; S <= (fs ? fs : std::max(smin, 64)); ++S) {
      const long long kc = cdiv(cdiv(K, S), TPL) * TPL;
      if (S > smin && kc < 16 && !fs) break;
      const long long splits = cdiv(K, kc);
      if (ws_limit >= 0 && splits > 1 && splits * R * O * 4 > ws_limit) continue;
      const double cost = (double)cdiv(tiles * splits, cus) * (double)(kc + 6) * f +
                          (splits > 1 ? 4.0 + splits * slice : 0.0);
      if (!found || cost < best_cost) {
        best_kc = kc; best_cost = cost; best_rt = rt; found = true;
      }
    }
  }
  if (!found) { pl.splits = -1; pl.k_chunk = 1; return pl; }
  pl.k_chunk = (int)std::min<long long>(best_kc, kmax);
  pl.splits = (int)cdiv(K, pl.k_chunk);
  // stream-K at the default rows per tile, when forced or cheaper
  const long long tiles = (long long)pl.tiles_r * pl.tiles_o;
  const bool split_only = (sched && !strcmp(sched, "split")) || force_rows || force_s;
  if (!split_only && K <= kmax && tiles % cus != 0 && (ws_limit < 0 || SK_SLOT_BYTES <= ws_limit)) {
    const long long rounds = tiles / cus;
    const long long tail = tiles - rounds * cus;
    const long long T = tail * pl.nqt;
    const long long per = cdiv(T, cus);
    if (per >= 2) {
      const long long cuts = std::min<long long>(tail, cdiv(T, per) - 1);
      const double sk_cost = (double)rounds * (K + 14) + 4.0 * per +
                             14.0 * (double)(cdiv(per, pl.nqt) + 1) +
                             (upper ? 0.7 : 0.1) * cuts + 45.0;
      if (force_sk || sk_cost < best_cost) {
        pl.sk_per = (int)per;
        pl.sk_dp = (int)(rounds * cus);
        return pl;                       // default rows per tile
      }
    }
  }
  pl.rt = best_rt;
  pl.tiles_r = R > 0 ? (int)cdiv(R, best_rt) : pl.tiles_r;
  return pl;
}

// ------------------------------------------------ no-allocation scratch
// Device memory of atx_lut_gemm_noalloc: a file-scope array, one copy per GPU
// for the life of the process.  Host code never uses its name as an address:
// the device address of this GPU's copy comes from hipGetSymbolAddress (with
// that device current) and is cached per device.
static __device__ __align__(256) unsigned char scratch[ATX_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_addr[MAX_DEVICES];

// Address of the current device's scratch array; the stream must belong to
// the current device (the address is only valid there).
static int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(ATX_ELAUNCH, "atx_lut_gemm_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= MAX_DEVICES)
    return set_error(ATX_ERANGE, "atx_lut_gemm_noalloc: device %d out of range", dev);
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess)
      return set_error(ATX_ELAUNCH, "atx_lut_gemm_noalloc: hipStreamGetDevice: %s",
                       hipGetErrorString(e));
    if (sdev != dev)
      return set_error(ATX_EINVAL,
                       "atx_lut_gemm_noalloc: the stream belongs to device %d, the current "
                       "device is %d", sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(ATX_ELAUNCH, "atx_lut_gemm_noalloc: hipGetSymbolAddress: %s",
                       hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return ATX_OK;
}

}  // namespace atx

using namespace atx;

extern "C" {

int atx_lut_prepare(const float* lut, uint16_t* out16t, float* outf32t,
                    int* flags, hipStream_t stream) {
  ATX_REQUIRE(lut && out16t && outf32t && flags, "atx_lut_prepare: null pointer");
  hipLaunchKernelGGL(lut_prepare_kernel, dim3(256), dim3(256), 0, stream, lut,
                     out16t, outf32t, flags);
  return check_launch("lut_prepare_kernel");
}

int atx_pack_x_f32(const float* x, int N, int K, int L, int offset, uint8_t* xq,
                   uint16_t* xt, int Rpad, int* upper, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0, "atx_pack_x_f32: negative size");
  ATX_REQUIRE(Rpad >= (long long)N * L && Rpad % RT == 0,
              "atx_pack_x_f32: Rpad must be a multiple of %d covering N*L", RT);
  if ((long long)K * Rpad == 0) return ATX_OK;
  // an empty x (N*L == 0) only writes the zero padding rows
  ATX_REQUIRE(xt && ((long long)N * L == 0 || x), "atx_pack_x_f32: null pointer");
  dim3 grid((unsigned)std::min<long long>(cdiv(Rpad / 4, 256), 1024),
            (unsigned)std::min(operand_rows(K), 65535));
  const bool vec = L % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)xq % 4 == 0;
  hipLaunchKernelGGL(pack_x_kernel<float>, grid, dim3(256), 0, stream, x, N, K, L,
                     offset, xq, xt, Rpad, vec, upper);
  return check_launch("pack_x_kernel<float>");
}

int atx_pack_x_u8(const uint8_t* xq, int N, int K, int L, uint16_t* xt, int Rpad,
                  int* upper, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0, "atx_pack_x_u8: negative size");
  ATX_REQUIRE(Rpad >= (long long)N * L && Rpad % RT == 0,
              "atx_pack_x_u8: Rpad must be a multiple of %d covering N*L", RT);
  if ((long long)K * Rpad == 0) return ATX_OK;
  ATX_REQUIRE(xt && ((long long)N * L == 0 || xq), "atx_pack_x_u8: null pointer");
  ATX_REQUIRE(operand_rows(K) / 4 <= 65535, "atx_pack_x_u8: K too large");
  const dim3 grid((unsigned)cdiv(Rpad / 4, 256), (unsigned)(operand_rows(K) / 4));
  const bool vec = L % 4 == 0 && (uintptr_t)xq % 4 == 0;
  hipLaunchKernelGGL(pack_x_u8_quads_kernel, grid, dim3(256), 0, stream, xq, N, K, L, xt, Rpad,
                     vec, upper);
  return check_launch("pack_x_u8_quads_kernel");
}

int atx_pack_w_f32(const float* w, int O, int K, int offset, uint8_t* wq,
                   uint8_t* wt, int Opad, hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && K >= 0, "atx_pack_w_f32: negative size");
  ATX_REQUIRE(Opad >= O && Opad % OT == 0,
              "atx_pack_w_f32: Opad must be a multiple of %d covering O", OT);
  if ((long long)K * Opad == 0) return ATX_OK;
  // an empty w (O == 0) only writes the padding columns
  ATX_REQUIRE((wt || wq) && (O == 0 || w), "atx_pack_w_f32: null pointer");
  hipLaunchKernelGGL(pack_w_kernel<float>, dim3(elem_grid((long long)K * Opad, 256)),
                     dim3(256), 0, stream, w, O, K, offset, wq, wt, Opad);
  return check_launch("pack_w_kernel<float>");
}

int atx_pack_w_u8(const uint8_t* wq, int O, int K, uint8_t* wt, int Opad,
                  hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && K >= 0, "atx_pack_w_u8: negative size");
  ATX_REQUIRE(Opad >= O && Opad % OT == 0,
              "atx_pack_w_u8: Opad must be a multiple of %d covering O", OT);
  if ((long long)K * Opad == 0) return ATX_OK;
  ATX_REQUIRE(wt && (O == 0 || wq), "atx_pack_w_u8: null pointer");
  hipLaunchKernelGGL(pack_w_kernel<uint8_t>, dim3(elem_grid((long long)K * Opad, 256)),
                     dim3(256), 0, stream, wq, O, K, 0, (uint8_t*)nullptr, wt, Opad);
  return check_launch("pack_w_kernel<u8>");
}

int atx_pack_rows_strided(const void* x, int dtype, int R, int K, long long sr, long long sk,
                          int offset, uint8_t* xq, uint16_t* xt, int Rpad, int* upper,
                          hipStream_t stream) {
  ATX_REQUIRE(R >= 0 && K >= 0 && (dtype == 0 || dtype == 1),
              "atx_pack_rows_strided: bad arguments");
  ATX_REQUIRE(Rpad >= R && Rpad % RT == 0,
              "atx_pack_rows_strided: Rpad must be a multiple of %d covering R", RT);
  if ((long long)K * Rpad == 0) return ATX_OK;
  ATX_REQUIRE(xt && (R == 0 || x), "atx_pack_rows_strided: null pointer");
  dim3 grid((unsigned)std::min<long long>(cdiv(Rpad / 4, 256), 1024),
            (unsigned)std::min(operand_rows(K), 65535));
  if (dtype == 0)
    hipLaunchKernelGGL(pack_rows_strided_kernel<float>, grid, dim3(256), 0, stream,
                       (const float*)x, R, K, sr, sk, offset, xq, xt, Rpad, upper);
  else
    hipLaunchKernelGGL(pack_rows_strided_kernel<uint8_t>, grid, dim3(256), 0, stream,
                       (const uint8_t*)x, R, K, sr, sk, 0, xq, xt, Rpad, upper);
  return check_launch("pack_rows_strided_kernel");
}

int atx_pack_cols_strided(const void* y, int dtype, int C, int K, long long sc, long long sk,
                          int offset, uint8_t* yq, uint8_t* wt, int Opad, hipStream_t stream) {
  ATX_REQUIRE(C >= 0 && K >= 0 && (dtype == 0 || dtype == 1),
              "atx_pack_cols_strided: bad arguments");
  ATX_REQUIRE(Opad >= C && Opad % OT == 0,
              "atx_pack_cols_strided: Opad must be a multiple of %d covering C", OT);
  if ((long long)K * Opad == 0) return ATX_OK;
  ATX_REQUIRE(wt && (C == 0 || y), "atx_pack_cols_strided: null pointer");
  const dim3 grid(elem_grid((long long)K * Opad, 256));
  if (dtype == 0)
    hipLaunchKernelGGL(pack_cols_strided_kernel<float>, grid, dim3(256), 0, stream,
                       (const float*)y, C, K, sc, sk, offset, yq, wt, Opad);
  else
    hipLaunchKernelGGL(pack_cols_strided_kernel<uint8_t>, grid, dim3(256), 0, stream,
                       (const uint8_t*)y, C, K, sc, sk, 0, yq, wt, Opad);
  return check_launch("pack_cols_strided_kernel");
}

long long atx_lut_gemm_workspace_bytes(int N, int K, int L, int O) {
  if (N <= 0 || K <= 0 || L <= 0 || O <= 0) return 0;
  // the launch plans with or without an x_upper flag: enough for either
  long long bytes = 0;
  for (int upper = 0; upper < 2; ++upper) {
    const Plan pl = make_plan(N, K, L, O, KMAX_U16, -1, upper != 0);
    if (pl.sk_per > 0) bytes = std::max(bytes, SK_SLOT_BYTES);
    else if (pl.splits > 1) bytes = std::max(bytes, (long long)pl.splits * N * O * L * 4);
  }
  return bytes;
}

}  // extern "C"

namespace atx {

// The body of atx_lut_gemm / atx_lut_gemm_noalloc.  ws_limit < 0: the
// workspace holds atx_lut_gemm_workspace_bytes() (caller-sized); otherwise
// the plan is restricted to schedules whose workspace fits ws_limit bytes,
// and `scratch()` supplies it (called only when a launch needs it).
template <typename ScratchFn>
static int lut_gemm_run(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad, int N, int K,
                        int L, int O, const uint16_t* lut16t, const float* lutf32t,
                        int lut_class, atx_gemm_epilogue ep, void* y, void* workspace,
                        long long ws_limit, ScratchFn scratch, hipStream_t stream) {
  ATX_REQUIRE_EPILOGUE(ep, "atx_lut_gemm");
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0 && O >= 0, "atx_lut_gemm: negative size");
  const long long R = (long long)N * L;
  ATX_REQUIRE(R <= 0x7fffffffLL - RT, "atx_lut_gemm: N*L too large");
  ATX_REQUIRE(Rpad >= R && Rpad % RT == 0, "atx_lut_gemm: bad Rpad %d", Rpad);
  // Four k-rows of the row-offset operand are addressed with 32-bit offsets.
  if ((long long)Rpad > (1LL << 27))
    return set_error(ATX_ERANGE, "atx_lut_gemm: Rpad %d exceeds 2^27 rows", Rpad);
  ATX_REQUIRE(Opad >= O && Opad % OT == 0, "atx_lut_gemm: bad Opad %d", Opad);
  ATX_REQUIRE(ep.out_kind >= ATX_OUT_F32 && ep.out_kind <= ATX_OUT_DEQUANT,
              "atx_lut_gemm: bad out_kind");
  ATX_REQUIRE(lut_class >= ATX_LUT_I16 && lut_class <= ATX_LUT_F32,
              "atx_lut_gemm: bad lut_class");
  ATX_REQUIRE(!(lut_class == ATX_LUT_F32 && ep.out_kind == ATX_OUT_I32),
              "atx_lut_gemm: int32 output needs an integer LUT");
  ATX_REQUIRE(ep.out_kind != ATX_OUT_DEQUANT || (ep.scale_x && ep.scale_w),
              "atx_lut_gemm: dequant epilogue needs scale_x and scale_w");
  if (R * O == 0) return ATX_OK;
  ATX_REQUIRE(y, "atx_lut_gemm: null output");
  // K == 0 is an empty contraction: every sum is 0 and only the epilogue runs.
  ATX_REQUIRE(K == 0 || (xt && wt), "atx_lut_gemm: null operand");

  GemmParams p{};
  p.xt = xt; p.Rpad = Rpad; p.wt = wt; p.Opad = Opad;
  p.lut16t = lut16t; p.lutf32t = lutf32t;
  p.K = K; p.R = (int)R; p.L = L; p.O = O;
  p.out_kind = ep.out_kind; p.y = y;
  p.sx = ep.scale_x; p.sw = ep.scale_w; p.bias = ep.bias;
  p.x_upper = ep.x_upper;

  if (lut_class == ATX_LUT_F32) {
    ATX_REQUIRE(lutf32t, "atx_lut_gemm: fp32 class needs the fp32 image");
    int rc = timing_mark(false, stream);
    if (rc == ATX_OK)
      rc = lut_gemm_f32_tiled(xt, Rpad, wt, Opad, lutf32t, N, K, L, O, ep.out_kind, ep.scale_x,
                              ep.scale_w, ep.bias, (float*)y, stream);
    return rc == ATX_OK ? timing_mark(true, stream) : rc;
  }
  ATX_REQUIRE(lut16t, "atx_lut_gemm: integer class needs the 16-bit image");
  const Plan pl = make_plan(N, K, L, O, KMAX_U16, ws_limit, ep.x_upper != nullptr);
  if (pl.splits < 0)
    return set_error(ATX_ERANGE,
                     "atx_lut_gemm_noalloc: K = %d needs %lld bytes of int32 partial sums "
                     "(R = %lld rows x O = %d), more than the %lld-byte scratch buffer; "
                     "call atx_lut_gemm with a workspace", K,
                     (long long)cdiv(K, KMAX_U16) * R * O * 4, R, O, ws_limit);
  if (ws_limit >= 0 && (pl.sk_per > 0 || pl.splits > 1)) {
    const int rc = scratch(&workspace);
    if (rc != ATX_OK) return rc;
  }
  p.tiles_r = pl.tiles_r; p.tiles_o = pl.tiles_o; p.rt = pl.rt;
  p.splits = pl.splits; p.k_chunk = pl.k_chunk;
  const long long numel = R * O;
  if (pl.sk_per > 0) {
    ATX_REQUIRE(workspace, "atx_lut_gemm: stream-K plan needs a workspace of %lld bytes",
                (long long)(PLAN_CUS - 1) * RT * OT * 4);
    p.sk_per = pl.sk_per; p.nqt = pl.nqt; p.skws = (int*)workspace;
    p.sk_dp = pl.sk_dp; p.sk_g = PLAN_CUS;
    p.splits = 1;
    const long long T = ((long long)pl.tiles_r * pl.tiles_o - pl.sk_dp) * pl.nqt;
    const unsigned Gt = (unsigned)cdiv(T, pl.sk_per);         // tail workgroups, <= PLAN_CUS
    const unsigned G = pl.sk_dp > 0 ? (unsigned)PLAN_CUS : Gt;
    if (Gt > 1) {
      hipLaunchKernelGGL(sk_clear_kernel, dim3(Gt - 1), dim3(NT), 0, stream, p);
      int rc = check_launch("sk_clear_kernel");
      if (rc != ATX_OK) return rc;
    }
    int rc = timing_mark(false, stream);
    if (rc != ATX_OK) return rc;
    if (lut_class == ATX_LUT_I16)
      hipLaunchKernelGGL(lut_gemm_kernel<true>, dim3(G), dim3(NT), 0, stream, p);
    else
      hipLaunchKernelGGL(lut_gemm_kernel<false>, dim3(G), dim3(NT), 0, stream, p);
    rc = check_launch("lut_gemm_kernel");
    if (rc == ATX_OK) rc = timing_mark(true, stream);
    if (rc != ATX_OK || Gt <= 1) return rc;
    hipLaunchKernelGGL(sk_finish_kernel, dim3(Gt - 1), dim3(NT), 0, stream, p);
    return check_launch("sk_finish_kernel");
  }
  if (pl.splits > 1) {
    ATX_REQUIRE(workspace, "atx_lut_gemm: split-K plan needs a workspace of %lld bytes",
                (long long)pl.splits * numel * 4);
    p.y = workspace;
    p.split_stride = numel;
  }
  const long long blocks = (long long)pl.tiles_r * pl.tiles_o * pl.splits;
  ATX_REQUIRE(blocks < 0x7fffffffLL, "atx_lut_gemm: grid too large");
  int rc = timing_mark(false, stream);
  if (rc != ATX_OK) return rc;
  if (lut_class == ATX_LUT_I16)
    hipLaunchKernelGGL(lut_gemm_kernel<true>, dim3((unsigned)blocks), dim3(NT), 0,
                       stream, p);
  else
    hipLaunchKernelGGL(lut_gemm_kernel<false>, dim3((unsigned)blocks), dim3(NT), 0,
                       stream, p);
  rc = check_launch("lut_gemm_kernel");
  if (rc == ATX_OK) rc = timing_mark(true, stream);
  if (rc != ATX_OK || pl.splits == 1) return rc;
  return launch_split_reduce((const int*)workspace, pl.splits, numel, O, L, ep, y, stream);
}

int launch_split_reduce(const int* ws, int S, long long numel, int O, int L,
                        const atx_gemm_epilogue& ep, void* y, hipStream_t stream,
                        const U8Terms& u8) {
  if (numel % 4 == 0 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)ws & 15) == 0)
    hipLaunchKernelGGL(split_reduce_kernel, dim3(elem_grid(numel / 4, 256)), dim3(256), 0,
                       stream, ws, S, numel, O, L, ep.out_kind, y, ep.scale_x, ep.scale_w,
                       ep.bias, u8);
  else
    hipLaunchKernelGGL(split_reduce1_kernel, dim3(elem_grid(numel, 256)), dim3(256), 0,
                       stream, ws, S, numel, O, L, ep.out_kind, y, ep.scale_x, ep.scale_w,
                       ep.bias, u8);
  return check_launch("split_reduce_kernel");
}

}  // namespace atx

extern "C" {

int atx_lut_gemm(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                 int N, int K, int L, int O, const uint16_t* lut16t,
                 const float* lutf32t, int lut_class, atx_gemm_epilogue ep,
                 void* y, void* workspace, hipStream_t stream) {
  return lut_gemm_run(xt, Rpad, wt, Opad, N, K, L, O, lut16t, lutf32t, lut_class, ep, y,
                      workspace, -1, [](void**) { return ATX_OK; }, stream);
}

int atx_lut_gemm_noalloc(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                         int N, int K, int L, int O, const uint16_t* lut16t,
                         const float* lutf32t, int lut_class, atx_gemm_epilogue ep,
                         void* y, hipStream_t stream) {
  return lut_gemm_run(xt, Rpad, wt, Opad, N, K, L, O, lut16t, lutf32t, lut_class, ep, y,
                      nullptr, ATX_NOALLOC_SCRATCH_BYTES,
                      [stream](void** ws) { return noalloc_scratch(stream, ws); }, stream);
}

}  // extern "C"
