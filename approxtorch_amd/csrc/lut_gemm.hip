// LUT GEMM forward for gfx950: y[n,o,l] = sum_k LUT[xi(n,k,l)][wi(o,k)].
//
// Kernel structure ("expanded tables"):
//   A workgroup owns a tile of ATX_ROW_TILE (1024) rows r = n*L + l and
//   ATX_COL_TILE (64) output channels.  For every k it builds, in LDS, the
//   table E_k[v][o] = LUT16[v][wi(o,k)] (256 rows x 64 channels x 16 bit =
//   32 KiB) from the transposed 16-bit LUT image (L2-resident, 128 KiB), then
//   every lane looks up E_k[xi(r,k)][o..o+7] for its rows with one
//   conflict-free 16-byte LDS read and adds the eight 16-bit entries into
//   int32 accumulators (exact).  Four E buffers (128 KiB of LDS) let each
//   step write the table two steps ahead, with one barrier per two steps.
//
//   LDS bank layout: an E row is 128 bytes (all 32 banks).  Its 16-byte
//   chunk for channels 8g..8g+7 is stored at chunk position g ^ ((v>>1)&7).
//   The activation operand is pre-encoded as the byte offset
//   v*128 + ((v>>1)&7)*16 ("row offset"), so the lane's address is
//   row_offset ^ (g*16): no arithmetic on the index itself.
//
//   Table build: wave w builds channel group w.  Its eight weight indices at
//   k are wave-uniform (one vector load read back with v_readlane); lane t
//   loads the dwords
//   LUT16T[w_j][2t, 2t+1] of the eight channels j (scalar base + lane
//   offset, 256 contiguous bytes per instruction), interleaves them with
//   v_perm into the 16-byte chunks of rows 2t and 2t+1 and stores each with
//   one ds_write_b128.  The swizzle gives the eight lanes of every write
//   group distinct chunk positions, so the writes are conflict-free (4-byte
//   LDS writes reach only about a third of the 16-byte write bandwidth).
//
//   Threads: 512 (8 waves).  Lane = (row group rg 0..7, channel group g);
//   wave w owns rows 128w .. 128w+127 of the tile and lane (rg, g) the rows
//   32h + 4rg + m (h, m = 0..3) x 8 channels = 128 int32 accumulators
//   (256-VGPR budget at 2 waves per SIMD).  Four consecutive rows per lane
//   let the epilogue store every (channel, h) as one 16-byte vector, and the
//   eight row groups of a channel fill a 128-byte line, so results go from
//   registers straight to HBM with all waves storing at once.
//
// Reference: bgemm_lut_u8_kernel / bgemm_mainloop
// (csrc/claude/bgemm_lut_kernels.cuh:183-387) computes the same sum with a
// 16-bit LUT gathered through L1 and fp32 accumulation.

#include "atx_internal.h"

#include <algorithm>
#include <type_traits>

namespace atx {

constexpr int RT = ATX_ROW_TILE;   // rows per workgroup
constexpr int OT = ATX_COL_TILE;   // channels per workgroup
#ifndef ATX_LUT_RPL
#define ATX_LUT_RPL 16
#endif
constexpr int RPL = ATX_LUT_RPL;   // rows per lane (16: 8 waves, 8: 16 waves)
constexpr int RPW = 8 * RPL;       // rows per wave (8 row groups)
constexpr int NWAVE = RT / RPW;    // waves per workgroup
constexpr int NT = 64 * NWAVE;     // threads per workgroup
constexpr int IPT = 1024 / NT;     // table-build items per thread
constexpr int ETAB = 256 * OT * 2; // bytes of one E_k table (32 KiB)
constexpr int NBUF = 4;                       // E tables resident in LDS
constexpr int SMEM_BYTES = NBUF * ETAB;       // 128 KiB of static LDS
constexpr int RQ = 4;              // consecutive rows per lane quad
constexpr int NQ = RPL / RQ;       // quads per lane (stride 32 rows)
static_assert(1024 % NT == 0, "table build needs an integral item count");
static_assert(RPW == 8 * RQ * NQ, "a wave's rows are 8 row groups x NQ quads");

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
  int out_kind;                 // ATX_OUT_*; splits > 1 => raw int32 partials
  void* y;
  long long split_stride;       // elements per partial slice
  const float* sx; const float* sw; const float* bias;
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
// xt[k][r] for r < R from x[n][k][l] (r = n*L + l); zero offsets for r >= R.
template <typename T>
__global__ void pack_x_kernel(const T* __restrict__ x, int N, int K, int L,
                              int offset, uint8_t* __restrict__ xq,
                              uint16_t* __restrict__ xt, int Rpad) {
  const int R = N * L;
  for (int k = blockIdx.y; k < K; k += gridDim.y) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < Rpad;
         r += gridDim.x * blockDim.x) {
      unsigned off = 0;
      if (r < R) {
        const int n = r / L;
        const int l = r - n * L;
        const long long src = ((long long)n * K + k) * L + l;
        unsigned v;
        if constexpr (sizeof(T) == 4) {
          v = quant_index((float)x[src], offset);
          if (xq) xq[src] = (uint8_t)v;
        } else {
          v = (unsigned)x[src];
        }
        off = row_offset(v);
      }
      xt[(long long)k * Rpad + r] = (uint16_t)off;
    }
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
    wt[i] = (uint8_t)v;
  }
}

// ------------------------------------------------------------- main kernel
__device__ __forceinline__ int logical_block() {
  // Blocks are dispatched round-robin over the 8 XCDs (bid % 8).  Give each
  // XCD a contiguous range of logical tiles so tiles sharing an activation
  // row tile (consecutive logical ids) share that XCD's L2.
  const int bid = blockIdx.x, nb = gridDim.x;
  const int q = nb >> 3, rem = nb & 7;
  const int xcd = bid & 7, slot = bid >> 3;
  return xcd < rem ? xcd * (q + 1) + slot : rem * (q + 1) + (xcd - rem) * q + slot;
}

template <bool SIGNED>
__device__ __forceinline__ void add8(int (&a)[8], const uint4 e) {
  const unsigned d[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (SIGNED) {
      a[2 * i] += (int)(short)(unsigned short)(d[i] & 0xffffu);
      a[2 * i + 1] += ((int)d[i]) >> 16;
    } else {
      a[2 * i] += (int)(d[i] & 0xffffu);
      a[2 * i + 1] += (int)(d[i] >> 16);
    }
  }
}

// Table-build registers: for each build item, the LUT16T dwords
// (entries v0, v0+1) of the wave's eight channels.
struct Rows { unsigned d[IPT][8]; };
// Row offsets of the lane's quads: v[h] = rows 32h + 4rg + 0..3, two per dword.
struct XRows { uint2 v[NQ]; };

// Raw buffer descriptor (word 3 of the gfx9-family descriptor: 32-bit
// elements, no swizzle) over `bytes` bytes at a wave-uniform base.  Buffer
// loads take the per-step offsets in scalar registers, so the loads below
// cost no per-lane 64-bit address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes,
                                           0x00020000);
}

// Eight weight indices (channels o0 + 8*og .. +7) at k, wcol = &wt[k][o0 +
// 8*og].  Lane parity picks the dword (indices 0-3 / 4-7) so the load is a
// vector load: a scalar load would share the LDS wait counter and,
// completing out of order, force every LDS wait of the step to drain it.
__device__ __forceinline__ unsigned load_w8(const uint8_t* wcol, int lane) {
  return __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(wcol, 8), (lane & 1) * 4, 0, 0);
}

// Dword at entries (v0, v0+1) of LUT16T row w_j for every channel j of the
// group; item i covers v0 = 2*lane + 128*i + sbase/2.  Row offsets are
// wave-uniform (read from lanes 0 and 1 of the weight-index register).
__device__ __forceinline__ void load_rows(Rows& r, __amdgpu_buffer_rsrc_t lut, unsigned wv,
                                          int lane, int sbase) {
  const unsigned w_lo = __builtin_amdgcn_readlane(wv, 0);
  const unsigned w_hi = __builtin_amdgcn_readlane(wv, 1);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const unsigned wj = ((j < 4 ? w_lo : w_hi) >> (8 * (j & 3))) & 255u;
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      r.d[i][j] = __builtin_amdgcn_raw_buffer_load_b32(lut, lane * 4 + 256 * i,
                                                        (int)(wj * 512u) + sbase, 0);
  }
}

// Row offsets of the lane's quads at k from the tile's row-offset column
// (xcol = &xt[k][first row of the tile]); xoff = byte offset of the lane's
// first quad within the tile.
__device__ __forceinline__ void load_x(XRows& x, const uint16_t* xcol, int xoff) {
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(xcol, RT * 2);
#pragma unroll
  for (int h = 0; h < NQ; ++h)
    x.v[h] = __builtin_bit_cast(
        uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, xoff + 16 * RQ * h, 0, 0));
}

// Writes this lane's two 16-byte chunks per build item (rows v0 and v0+1,
// channels 8*og .. 8*og+7); wbase holds the chunk address of row v0 within
// the table at smem.
__device__ __forceinline__ void write_table(unsigned char* smem, const Rows& r,
                                            const int (&wbase)[IPT]) {
#pragma unroll
  for (int it = 0; it < IPT; ++it) {
    const unsigned* d = r.d[it];
    uint4 lo, hi;      // channel pairs (2m, 2m+1) at v0 (low halves) / v0+1 (high)
    lo.x = __builtin_amdgcn_perm(d[1], d[0], 0x05040100u);
    lo.y = __builtin_amdgcn_perm(d[3], d[2], 0x05040100u);
    lo.z = __builtin_amdgcn_perm(d[5], d[4], 0x05040100u);
    lo.w = __builtin_amdgcn_perm(d[7], d[6], 0x05040100u);
    hi.x = __builtin_amdgcn_perm(d[1], d[0], 0x07060302u);
    hi.y = __builtin_amdgcn_perm(d[3], d[2], 0x07060302u);
    hi.z = __builtin_amdgcn_perm(d[5], d[4], 0x07060302u);
    hi.w = __builtin_amdgcn_perm(d[7], d[6], 0x07060302u);
    *(uint4*)(smem + wbase[it]) = lo;
    *(uint4*)(smem + wbase[it] + 128) = hi;
  }
}

// Accumulates one table for this lane's RPL rows.  x holds the rows'
// offsets (two per dword, below 32768); gx XORs in the lane's channel chunk
// (bits 4-6) and possibly bit 16 of the table's LDS address.
template <bool SIGNED>
__device__ __forceinline__ void use_table(int (&acc)[RPL][8], const unsigned char* smem,
                                          const XRows& x, unsigned gx) {
  // Reads per batch: 8 (two quads) at 2 waves per SIMD, 4 (one quad) at 4
  // waves per SIMD, where the register budget is half as large.
  constexpr int QB = RPL >= 16 ? 2 : 1;
#pragma unroll
  for (int hh = 0; hh < NQ; hh += QB) {
    unsigned xd[2 * QB];
#pragma unroll
    for (int q = 0; q < QB; ++q) { xd[2 * q] = x.v[hh + q].x; xd[2 * q + 1] = x.v[hh + q].y; }
    uint4 e[4 * QB];
#pragma unroll
    for (int j = 0; j < 2 * QB; ++j) {
      e[2 * j] = *(const uint4*)(smem + ((xd[j] & 0xffffu) ^ gx));
      e[2 * j + 1] = *(const uint4*)(smem + ((xd[j] >> 16) ^ gx));
    }
#pragma unroll
    for (int j = 0; j < 4 * QB; ++j) add8<SIGNED>(acc[RQ * hh + j], e[j]);
    if constexpr (QB == 1) __builtin_amdgcn_sched_barrier(0);
  }
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

// Smallest entry of the waves' progress slots (wave-uniform).
__device__ __forceinline__ unsigned min_progress(const unsigned* prog) {
  static_assert(NWAVE % 4 == 0, "16-byte reads cover the slots");
  unsigned m = ~0u;
#pragma unroll
  for (int i = 0; i < NWAVE / 4; ++i) {
    const uint4 a = *(const uint4*)(prog + 4 * i);
    m = min(m, min(min(a.x, a.y), min(a.z, a.w)));
  }
  return __builtin_amdgcn_readfirstlane(m);
}

// Writes the lane's accumulators: channel o0 + e, rows r + 32h + m of quad
// h (r = first row of quad 0).  Rows beyond R and channels beyond O are
// dropped.  With L % 4 == 0 a quad never straddles two images and is one
// 16-byte store (r is a multiple of 4); otherwise rows are stored one by one,
// stepping (n, l) across image boundaries.
template <int KIND>
__device__ __forceinline__ void store_tile(const GemmParams& p, void* y,
                                           const int (&acc)[RPL][8], int r, int o0) {
  const bool vec = (p.L & 3) == 0;
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    const int rq = r + 8 * RQ * h;
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

template <bool SIGNED>
__global__ void __launch_bounds__(NT, 1)
lut_gemm_kernel(const GemmParams p) {
  __shared__ __align__(16) unsigned char smem[SMEM_BYTES];
  __shared__ __align__(16) unsigned progress[NWAVE];   // k-steps finished per wave
  __shared__ unsigned pscratch[NT];    // branch-free progress store: other lanes' sink

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane >> 3, g = lane & 7;

  int lb = logical_block();
  const int to = lb % p.tiles_o; lb /= p.tiles_o;
  const int tr = lb % p.tiles_r;
  const int s = lb / p.tiles_r;

  const int o0 = to * OT;
  const int r0 = tr * RT + wave * RPW + rg * RQ;         // this lane's first quad
  const int kb = s * p.k_chunk;
  const int ke = min(p.K, kb + p.k_chunk);

  // Table-build mapping: wave w builds channel group og = w % 8 for rows
  // 128 hw .. 128 hw + 128 IPT - 1 (hw = w / 8); lane t writes rows
  // v0 = 2t + 128(i + hw) and v0+1 (item i), whose chunk og sits at position
  // og ^ ((v0 >> 1) & 7) = og ^ (t & 7).  Tables 0/1 and 2/3 of the four
  // LDS buffers differ by an immediate offset (0 / ETAB) from the base
  // addresses wlo / whi (whi = wlo + 2 * ETAB).
  static_assert((NWAVE == 8 && IPT == 2) || (NWAVE == 16 && IPT == 1),
                "eight channel groups x 256 rows per table");
  static_assert(NBUF == 4 && 2 * ETAB == 65536, "buffer pairs split at bit 16");
  const int og = __builtin_amdgcn_readfirstlane(wave & 7);
  const int hw = __builtin_amdgcn_readfirstlane(wave >> 3);
  int wlo[IPT], whi[IPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    wlo[i] = (2 * lane + 128 * (i + hw)) * 128 + ((og ^ (lane & 7)) << 4);
    whi[i] = wlo[i] + 2 * ETAB;
  }
  const unsigned gxa = (unsigned)(g << 4);              // reads of buffers 0, 1
  const unsigned gxb = gxa | (unsigned)(2 * ETAB);      // reads of buffers 2, 3

  const uint16_t* __restrict__ xtile = p.xt + (long long)tr * RT;
  const int xoff = (wave * RPW + rg * RQ) * 2;         // lane's first quad, bytes
  const uint8_t* __restrict__ wcol = p.wt + o0 + og * 8;
  const __amdgpu_buffer_rsrc_t lutr = buffer_rsrc(p.lut16t, 256 * 256 * 2);
  // Zero-length view of the image: its loads are out of range and return 0,
  // which builds an all-zero table for the steps past the chunk's end.
  const __amdgpu_buffer_rsrc_t lutz = buffer_rsrc(p.lut16t, 0);

  int acc[RPL][8];
#pragma unroll
  for (int j = 0; j < RPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0;

  if (tid < NWAVE) progress[tid] = 0u;   // ordered before use by the prologue barrier
  unsigned* const pslot = lane == 0 ? &progress[wave] : &pscratch[tid];

  if (kb < ke) {
    // Four LDS buffers, table t = k - kb in buffer t % 4.  Step t issues the
    // loads for row offsets t+1, LUT rows of table t+2 and weight indices of
    // t+3 (indices clamped to the range, so every load is unconditional),
    // accumulates from table t, writes table t+2 and records t+1 steps done
    // in its progress slot.  The loop is unrolled over the four buffers so
    // every buffer offset is an immediate and the row-offset registers
    // alternate between two sets without copies.
    //
    // Split barrier: instead of a workgroup barrier per step, a wave starts
    // step t once every wave has finished step t-2 (min over the progress
    // slots >= t-1).  That covers both hazards of the step: table t was
    // written in step t-2, and table t+2 reuses the buffer of table t-2,
    // last read in step t-2.  Waves may drift one step apart, which keeps
    // the VALU busy while other waves wait on LDS.  Buffers in use at once:
    // a slow wave at step t-1 holds tables t-1 and t+1, a fast wave at step
    // t tables t and t+2.  A wave's LDS operations execute in program
    // order, so its progress store lands after its table writes and its
    // reads of table t-2, and a wave that has seen the store issues its
    // table reads after that.  Every wave waits only for steps that it has
    // itself already finished, so the waits always end.  Compiler fences
    // keep the LDS accesses and the progress slots in program order;
    // scheduling fences keep the loads ahead of the accumulation and the
    // table write (which waits for the LUT rows) behind it, so the loads
    // overlap a whole step.
    const int klast = ke - 1;
    const long long xstride = p.Rpad, wstride = p.Opad;
    XRows xa, xb;
    unsigned wnext;                                         // indices of table t+2
    {
      const unsigned w0 = load_w8(wcol + kb * wstride, lane);
      const unsigned w1 = load_w8(wcol + min(kb + 1, klast) * wstride, lane);
      wnext = load_w8(wcol + min(kb + 2, klast) * wstride, lane);
      Rows rows;
      load_rows(rows, lutr, w0, lane, 256 * hw);
      load_x(xa, xtile + kb * xstride, xoff);
      write_table(smem, rows, wlo);                         // table kb   -> buffer 0
      load_rows(rows, ke - kb > 1 ? lutr : lutz, w1, lane, 256 * hw);
      write_table(smem + ETAB, rows, wlo);                  // table kb+1 -> buffer 1
    }
    __syncthreads();

    const unsigned n = (unsigned)(ke - kb);
    auto step = [&](auto bufc, unsigned t, XRows& xcur, XRows& xnext)
        __attribute__((always_inline)) {
      constexpr int B = decltype(bufc)::value;              // buffer of table t
      constexpr int BW = (B + 2) & 3;                       // buffer of table t+2
      const int k = kb + (int)t;
      load_x(xnext, xtile + min(k + 1, klast) * xstride, xoff);
      Rows rows;
      load_rows(rows, t + 2u < n ? lutr : lutz, wnext, lane, 256 * hw);
      const unsigned wn3 = load_w8(wcol + min(k + 3, klast) * wstride, lane);
      __builtin_amdgcn_sched_barrier(0);
      const unsigned need = t ? t - 1u : 0u;
      asm volatile("" ::: "memory");
      unsigned seen = min_progress(progress);
      while (seen < need) {
        __builtin_amdgcn_s_sleep(1);
        asm volatile("" ::: "memory");
        seen = min_progress(progress);
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      use_table<SIGNED>(acc, smem + (B & 1) * ETAB, xcur, (B & 2) ? gxb : gxa);
      // Pin the adds here: left free, the compiler sinks them into later
      // steps, past the table write that waits for this step's loads.
#pragma unroll
      for (int j = 0; j < RPL; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(acc[j][e]));
      __builtin_amdgcn_sched_barrier(0);
      write_table(smem + (BW & 1) * ETAB, rows, (BW & 2) ? whi : wlo);
      asm volatile("" ::: "memory");
      *pslot = t + 1u;          // lane 0: progress[wave]; others: scratch slots
      asm volatile("" ::: "memory");
      wnext = wn3;
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using B2 = std::integral_constant<int, 2>;
    using B3 = std::integral_constant<int, 3>;
    // Whole groups of four steps; the up to three steps past the chunk's
    // end accumulate all-zero tables (built from lutz), so the accumulation
    // needs no branch and every wave runs the same steps.
    for (unsigned t = 0; t < n; t += 4u) {
      step(B0{}, t, xa, xb);
      step(B1{}, t + 1u, xb, xa);
      step(B2{}, t + 2u, xa, xb);
      step(B3{}, t + 3u, xb, xa);
    }
  }

  // ---- epilogue: registers -> HBM, every wave at once (no LDS staging).
  const int oc = o0 + g * 8;
  if (p.splits > 1)
    store_tile<ATX_OUT_I32>(p, (int*)p.y + (long long)s * p.split_stride, acc, r0, oc);
  else if (p.out_kind == ATX_OUT_I32)
    store_tile<ATX_OUT_I32>(p, p.y, acc, r0, oc);
  else if (p.out_kind == ATX_OUT_F32)
    store_tile<ATX_OUT_F32>(p, p.y, acc, r0, oc);
  else
    store_tile<ATX_OUT_DEQUANT>(p, p.y, acc, r0, oc);
}

// Split-K reduction: exact int64 sum of int32 partials, then the epilogue.
__global__ void split_reduce_kernel(const int* __restrict__ ws, int S,
                                    long long numel, int O, int L, int out_kind,
                                    void* __restrict__ y, const float* sx,
                                    const float* sw, const float* bias) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < numel;
       i += (long long)gridDim.x * blockDim.x) {
    long long a = 0;
    for (int s = 0; s < S; ++s) a += ws[(long long)s * numel + i];
    if (out_kind == ATX_OUT_I32) {
      ((int*)y)[i] = (int)a;
    } else if (out_kind == ATX_OUT_F32) {
      ((float*)y)[i] = (float)a;
    } else {
      const int o = (int)((i / L) % O);
      const float sc = sx[0] * sw[o];
      const float t = (float)a * sc;
      ((float*)y)[i] = bias ? bias[o] + t : t;
    }
  }
}

// fp32-LUT fallback: one thread per output, fp32 sum in ascending k (the
// reference's non-split order, csrc/claude/bgemm_lut_kernels.cuh:276-284).
__global__ void lut_gemm_f32_kernel(const GemmParams p) {
  const long long numel = (long long)p.R * p.O;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < numel;
       i += (long long)gridDim.x * blockDim.x) {
    const int o = (int)(i / p.R);
    const int r = (int)(i - (long long)o * p.R);
    float a = 0.0f;
    for (int k = 0; k < p.K; ++k) {
      const unsigned xi = (unsigned)p.xt[(long long)k * p.Rpad + r] >> 7;
      const unsigned wi = p.wt[(long long)k * p.Opad + o];
      a += p.lutf32t[wi * 256u + xi];
    }
    const int n = r / p.L, l = r - (r / p.L) * p.L;
    const long long yi = ((long long)n * p.O + o) * p.L + l;
    if (p.out_kind == ATX_OUT_DEQUANT) {
      const float t = a * (p.sx[0] * p.sw[o]);
      ((float*)p.y)[yi] = p.bias ? p.bias[o] + t : t;
    } else {
      ((float*)p.y)[yi] = a;
    }
  }
}

// Split plan shared by the workspace query and the launch.
struct Plan { int tiles_r, tiles_o, splits, k_chunk; };

// Compute units of a full MI355X (one resident workgroup each: the kernel's
// 8 waves hold 2 waves per SIMD at its register budget).  A constant, not a
// device query, so the workspace query and the launch always agree.
constexpr int PLAN_CUS = 256;

// Split-K count by a cost model in units of one k-step of one workgroup:
//   ceil(tiles*S / CUs) rounds x (ceil(K/S) + 3 fixed steps per workgroup)
//   + for S > 1: 4 steps for the reduce launch and S x (R*O / 600000) steps
//     for writing and re-reading one int32 partial slice (8 bytes per
//     output at ~4 TB/s against ~1.2 us per k-step).
// S is at least ceil(K / kmax), the exact-int32 bound of one pass, and the
// smallest S among equal costs wins.
static Plan make_plan(int N, int K, int L, int O, int kmax) {
  Plan pl;
  const long long R = (long long)N * L;
  pl.tiles_r = (int)cdiv(R, RT);
  pl.tiles_o = (int)cdiv(O, OT);
  if (K <= 0) { pl.splits = 1; pl.k_chunk = 1; return pl; }
  const long long tiles = (long long)pl.tiles_r * pl.tiles_o;
  const long long cus = PLAN_CUS;
  const int smin = (int)cdiv(K, kmax);
  const double slice = (double)R * O / 600000.0;
  int best = smin;
  double best_cost = 0.0;
  for (int S = smin; S <= std::max(smin, 64); ++S) {
    const long long kc = cdiv(K, S);
    if (S > smin && kc < 16) break;
    const double cost = (double)cdiv(tiles * S, cus) * (double)(kc + 3) +
                        (S > 1 ? 4.0 + S * slice : 0.0);
    if (S == smin || cost < best_cost) { best = S; best_cost = cost; }
  }
  pl.k_chunk = (int)cdiv(K, best);
  pl.splits = (int)cdiv(K, pl.k_chunk);
  return pl;
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
                   uint16_t* xt, int Rpad, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0, "atx_pack_x_f32: negative size");
  ATX_REQUIRE(Rpad >= (long long)N * L && Rpad % RT == 0,
              "atx_pack_x_f32: Rpad must be a multiple of %d covering N*L", RT);
  if ((long long)K * Rpad == 0) return ATX_OK;
  // an empty x (N*L == 0) only writes the zero padding rows
  ATX_REQUIRE(xt && ((long long)N * L == 0 || x), "atx_pack_x_f32: null pointer");
  dim3 grid((unsigned)std::min<long long>(cdiv(Rpad, 256), 1024), (unsigned)std::min(K, 65535));
  hipLaunchKernelGGL(pack_x_kernel<float>, grid, dim3(256), 0, stream, x, N, K, L,
                     offset, xq, xt, Rpad);
  return check_launch("pack_x_kernel<float>");
}

int atx_pack_x_u8(const uint8_t* xq, int N, int K, int L, uint16_t* xt, int Rpad,
                  hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0, "atx_pack_x_u8: negative size");
  ATX_REQUIRE(Rpad >= (long long)N * L && Rpad % RT == 0,
              "atx_pack_x_u8: Rpad must be a multiple of %d covering N*L", RT);
  if ((long long)K * Rpad == 0) return ATX_OK;
  ATX_REQUIRE(xt && ((long long)N * L == 0 || xq), "atx_pack_x_u8: null pointer");
  dim3 grid((unsigned)std::min<long long>(cdiv(Rpad, 256), 1024), (unsigned)std::min(K, 65535));
  hipLaunchKernelGGL(pack_x_kernel<uint8_t>, grid, dim3(256), 0, stream, xq, N, K,
                     L, 0, (uint8_t*)nullptr, xt, Rpad);
  return check_launch("pack_x_kernel<u8>");
}

int atx_pack_w_f32(const float* w, int O, int K, int offset, uint8_t* wq,
                   uint8_t* wt, int Opad, hipStream_t stream) {
  ATX_REQUIRE(O >= 0 && K >= 0, "atx_pack_w_f32: negative size");
  ATX_REQUIRE(Opad >= O && Opad % OT == 0,
              "atx_pack_w_f32: Opad must be a multiple of %d covering O", OT);
  if ((long long)K * Opad == 0) return ATX_OK;
  // an empty w (O == 0) only writes the padding columns
  ATX_REQUIRE(wt && (O == 0 || w), "atx_pack_w_f32: null pointer");
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

long long atx_lut_gemm_workspace_bytes(int N, int K, int L, int O) {
  if (N <= 0 || K <= 0 || L <= 0 || O <= 0) return 0;
  const Plan pl = make_plan(N, K, L, O, KMAX_U16);
  if (pl.splits <= 1) return 0;
  return (long long)pl.splits * N * O * L * 4;
}

int atx_lut_gemm(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                 int N, int K, int L, int O, const uint16_t* lut16t,
                 const float* lutf32t, int lut_class, atx_gemm_epilogue ep,
                 void* y, void* workspace, hipStream_t stream) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0 && O >= 0, "atx_lut_gemm: negative size");
  const long long R = (long long)N * L;
  ATX_REQUIRE(R <= 0x7fffffffLL - RT, "atx_lut_gemm: N*L too large");
  ATX_REQUIRE(Rpad >= R && Rpad % RT == 0, "atx_lut_gemm: bad Rpad %d", Rpad);
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

  if (lut_class == ATX_LUT_F32) {
    ATX_REQUIRE(lutf32t, "atx_lut_gemm: fp32 class needs the fp32 image");
    p.tiles_r = p.tiles_o = p.splits = 1;
    hipLaunchKernelGGL(lut_gemm_f32_kernel, dim3(elem_grid(R * O, 256)), dim3(256),
                       0, stream, p);
    return check_launch("lut_gemm_f32_kernel");
  }
  ATX_REQUIRE(lut16t, "atx_lut_gemm: integer class needs the 16-bit image");
  const Plan pl = make_plan(N, K, L, O, KMAX_U16);
  p.tiles_r = pl.tiles_r; p.tiles_o = pl.tiles_o;
  p.splits = pl.splits; p.k_chunk = pl.k_chunk;
  const long long numel = R * O;
  if (pl.splits > 1) {
    ATX_REQUIRE(workspace, "atx_lut_gemm: split-K plan needs a workspace of %lld bytes",
                (long long)pl.splits * numel * 4);
    p.y = workspace;
    p.split_stride = numel;
  }
  const long long blocks = (long long)pl.tiles_r * pl.tiles_o * pl.splits;
  ATX_REQUIRE(blocks < 0x7fffffffLL, "atx_lut_gemm: grid too large");
  if (lut_class == ATX_LUT_I16)
    hipLaunchKernelGGL(lut_gemm_kernel<true>, dim3((unsigned)blocks), dim3(NT), 0,
                       stream, p);
  else
    hipLaunchKernelGGL(lut_gemm_kernel<false>, dim3((unsigned)blocks), dim3(NT), 0,
                       stream, p);
  int rc = check_launch("lut_gemm_kernel");
  if (rc != ATX_OK || pl.splits == 1) return rc;
  hipLaunchKernelGGL(split_reduce_kernel, dim3(elem_grid(numel, 256)), dim3(256), 0,
                     stream, (const int*)workspace, pl.splits, numel, O, L,
                     ep.out_kind, y, ep.scale_x, ep.scale_w, ep.bias);
  return check_launch("split_reduce_kernel");
}

}  // extern "C"
