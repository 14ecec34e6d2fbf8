// Custom (pair-wise 256x256 table) gradients of the LUT GEMM:
//   grad_x[n,k,l] = sum_o dy[n,o,l] * DX[xi(n,k,l)][wi(o,k)]
//   grad_w[o,k]   = sum_{n,l} dy[n,o,l] * DW[xi(n,k,l)][wi(o,k)]
// Reference: csrc/cuda/bgemm_custom_grad_optimize.cu:30-205 (uint8 indices),
// 315-490 (int8 values, index v+128): one output per thread, the table
// gathered through L1 (grad_x) or one column of it staged in shared memory
// per output (grad_w).
//
// Design (LDS-resident expanded tables, the LUT GEMM forward's layout in
// fp32).  A workgroup (512 threads, 8 waves) owns 2048 rows r = n*L + l; its
// lanes read the forward's row-offset operand xt [Kpad][Rpad] (no im2col of
// the saved image).  For a tap k and a tile of 16 channels o it builds the
// expanded table E[v][o] = T[v][wi(o,k)] (256 rows x 16 fp32 = 16 KiB) from
// the transposed table T^T (column wi contiguous, L2-resident), four tables
// to an LDS line with the quarter rotation of the forward, so every 16-byte
// read (four channels of one row) is conflict-free.  Lane (rg, g) owns 16
// rows and channels 4g..4g+3 of the tile; at sub-step s of a quad it handles
// tap 4j + ((rg + s) & 3) for all its rows (the operand's slot rotation).
//
//   grad_x: a workgroup owns a chunk of consecutive quads of taps and loops
//           over (quad, 16-channel tile) steps (tables of the next step built
//           while the current one is read); the 64 accumulators acc[s][row]
//           of a lane collect its four channels, and after a quad's last
//           channel tile the four lanes of a row group are summed with DPP
//           and stored.
//   grad_w: contracts over the rows.  L % 4 == 0: a workgroup keeps eight
//           taps' tables resident and walks a chunk of row steps, loading dy
//           per step (custom_dw_kernel).  Otherwise a workgroup owns one
//           16-channel tile of one row tile and streams all tap quads with
//           its dy in registers (custom_dw_tile_kernel).  Either way the
//           lane's partial sums are combined over the 16 row groups of a wave
//           with DPP (register indices chosen so every lane adds the same
//           tap), then over the waves through LDS, into one partial slice
//           per row chunk / row tile; the slices are summed in a fixed order.
// The table entries must be finite (padding rows of a partial row tile read
// table row 0 with dy = 0).
#include "atx_internal.h"
#include "atx_tiles.h"

#include <algorithm>
#include <type_traits>

#ifndef ATX_DW_WAVES
#define ATX_DW_WAVES 8           // waves per grad_w workgroup (resident tables)
#endif

namespace atx {
namespace cg {

using namespace tiles;
constexpr int RT = ATX_ROW_TILE;   // rows per workgroup (2048)
constexpr int CT = 16;             // channels per table tile
constexpr int NWAVE = RT / RPW;    // 8
constexpr int NT = 64 * NWAVE;     // 512 threads
constexpr int TPL = 4;             // tables per LDS line (quarters)
constexpr int LINE = 256;          // bytes per LDS line
constexpr int QTAB = 256 * LINE;   // one quad of tables (64 KiB)
constexpr int RED1 = NWAVE * 4 * 4 * 16;  // grad_w stage-1 floats per buffer (8 KiB)
constexpr int RED2 = NWAVE * 64;          // grad_w stage-2 floats per buffer (2 KiB)
static_assert(CT * 4 == LINE / TPL, "a table row fills one quarter of a line");

struct Params {
  const uint16_t* xt; int Rpad;
  const uint8_t* wt; int Opad;
  const float* tab;        // transposed pair table: tab[w * 256 + v] = T[v][w]
  const float* dy;         // [N][O][L]
  const float* dys;        // grad_w: per-channel factor of dy [O] (nullable)
  float* out;              // grad_x [N][K][L], or the grad_w slices [row chunks][O][K]
  int K, R, L, O;
  int tiles_r, tiles_o, nq; // nq = quads of taps
  int kq_chunk, kchunks;    // quads per workgroup, tap chunks
  int rchunk, rsteps;       // grad_w (resident tables): steps per workgroup, steps over R
};

// DPP helpers (quad_perm / row_shr controls of the VOP DPP encoding).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                       0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
constexpr int QP_XOR1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int QP_XOR2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int ROW_SHR4 = 0x114, ROW_SHR8 = 0x118, ROW_SHR12 = 0x11C;

// dy of the lane's rows for a run of channels, through a buffer descriptor
// over dy (its size is checked below 2^31 bytes on the host).  DyRows holds,
// per row quad h, the byte offset of dy[n][o_lane][l] for the quad's first
// row (o_lane = the lane's first channel of tile 0) or, for a quad at or past
// R, an offset beyond the buffer, which loads 0.  VEC (L % 4 == 0): a quad
// never straddles two images and is one 16-byte load per channel; otherwise
// each row of the quad has its own offset.
template <bool VEC>
struct DyRows { unsigned off[NQ][VEC ? 1 : RQ]; };

constexpr unsigned DY_OOB = 0x80000000u;

template <bool VEC>
__device__ __forceinline__ void dy_rows(const Params& p, int r0, int o_lane, DyRows<VEC>& d) {
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    const int rq = r0 + NRG * RQ * h;
    int n = rq / p.L, l = rq - n * p.L;
#pragma unroll
    for (int m = 0; m < (VEC ? 1 : RQ); ++m) {
      d.off[h][m] = rq + m < p.R
                        ? (unsigned)((((long long)n * p.O + o_lane) * p.L + l) * 4) : DY_OOB;
      if (++l == p.L) { l = 0; ++n; }
    }
  }
}

// dy of the lane's 16 rows for channels o_lane + ob .. + 3 (ob = tile base,
// wave-uniform); channels >= O load 0 (valid = number of the lane's four
// channels below O).
template <bool VEC>
__device__ __forceinline__ void load_dy(__amdgpu_buffer_rsrc_t dyr, const DyRows<VEC>& d, int L,
                                        int ob, int valid, float (&v)[RPL][4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int soff = (ob + c) * L * 4;
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      if constexpr (VEC) {
        const unsigned off = c < valid ? d.off[h][0] : DY_OOB;
        const float4 f = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(dyr, off, soff, 0));
        v[RQ * h][c] = f.x; v[RQ * h + 1][c] = f.y; v[RQ * h + 2][c] = f.z;
        v[RQ * h + 3][c] = f.w;
      } else {
#pragma unroll
        for (int m = 0; m < RQ; ++m)
          v[RQ * h + m][c] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(dyr, c < valid ? d.off[h][m] : DY_OOB,
                                                          soff, 0));
      }
    }
  }
}

// Table-build registers: the dwords T^T[w_c][v0], [v0 + 1] of the wave's four
// channels c (rows v0 = 128 hw + 2 lane and v0 + 1).
struct Src { float2 d[4]; };

// Four channel indices of the wave's group at tap k (one dword; a vector
// load, read back with v_readlane -- a scalar load in the loop would drain
// the LDS counter).
__device__ __forceinline__ unsigned load_w4(const uint8_t* wcol) {
  return __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(wcol, 4), 0, 0, 0);
}

__device__ __forceinline__ void load_src(Src& s, __amdgpu_buffer_rsrc_t tab, unsigned wv,
                                         int lane, int hw) {
  const unsigned w4 = __builtin_amdgcn_readfirstlane(wv);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const unsigned wc = (w4 >> (8 * c)) & 255u;
    s.d[c] = __builtin_bit_cast(
        float2, __builtin_amdgcn_raw_buffer_load_b64(tab, lane * 8, (int)(wc * 1024u) + hw * 512,
                                                     0));
  }
}

// Writes rows v0 and v0 + 1 (four channels each) of one table at smem + wb.
__device__ __forceinline__ void write_src(unsigned char* smem, const Src& s, int wb) {
  *(float4*)(smem + wb) = make_float4(s.d[0].x, s.d[1].x, s.d[2].x, s.d[3].x);
  *(float4*)(smem + wb + LINE) = make_float4(s.d[0].y, s.d[1].y, s.d[2].y, s.d[3].y);
}

// The pipelined table stream shared by both kernels: nsteps quads of four
// tables; table (step, s) is described by `col(step, s, og)` = pointer to the
// 4 channel indices of wave group og (wt[k][o0 + 4 og]).  `rows(x, step, s)`
// loads the lane's row offsets of sub-step s of quad `step`; `use(B, S, step,
// x)` consumes sub-step S of quad `step` from buffer B; `quad_end(step)` runs
// before each quad's closing barrier and `quad_begin(step)` right after the
// first sub-step's reads.
// Prefetch distances: row offsets two sub-steps ahead (four rotating
// buffers), channel indices two ahead of the table loads they address, the
// table entries one sub-step ahead of their LDS write.  Loads are issued
// oldest-consumer first (table entries, indices, row offsets), so the
// in-order vmcnt wait of each consumer never waits for a younger prefetch.
template <typename Col, typename Rows, typename Use, typename QEnd, typename QBegin>
__device__ __forceinline__ void table_stream(unsigned char* smem, const float* tab, int nsteps,
                                             Col col, Rows rows, Use use, QEnd quad_end,
                                             QBegin quad_begin) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int og = __builtin_amdgcn_readfirstlane(wave % 4);
  const int hw = __builtin_amdgcn_readfirstlane(wave / 4);
  const int wb0 = (128 * hw + 2 * lane) * LINE + ((og ^ (lane & 3)) << 4);
  const int wb1 = wb0 + QTAB;
  const __amdgpu_buffer_rsrc_t tabr = buffer_rsrc(tab, 256 * 256 * 4);
  const int last = 4 * nsteps - 1;
  auto colq = [&](int t) { return col(std::min(t, last) >> 2, std::min(t, last) & 3, og); };

  XRows xr[TPL];
  Src src;
  unsigned w1, w2;                                    // indices of tables sigma+5, sigma+6
  {
    Src s4;
#pragma unroll
    for (int q = 0; q < TPL; ++q) {
      load_src(s4, tabr, load_w4(colq(q)), lane, hw);
      write_src(smem + q * 64, s4, wb0);                 // quad 0 -> buffer 0
    }
    load_src(src, tabr, load_w4(colq(TPL)), lane, hw);
    w1 = load_w4(colq(TPL + 1));
    w2 = load_w4(colq(TPL + 2));
    rows(xr[0], 0, 0);
    rows(xr[1], 0, 1);
  }
  __syncthreads();

  auto sub = [&](auto bc, auto sc, int j) __attribute__((always_inline)) {
    constexpr int B = decltype(bc)::value;
    constexpr int S = decltype(sc)::value;
    const int sigma = TPL * j + S;
    Src sn;
    load_src(sn, tabr, w1, lane, hw);                    // table sigma + 5
    w1 = w2;
    w2 = load_w4(colq(sigma + 7));
    if constexpr (S + 2 < TPL) rows(xr[(S + 2) & 3], j, S + 2);
    else rows(xr[(S + 2) & 3], j + 1, S - 2);
    __builtin_amdgcn_sched_barrier(0);
    use(bc, sc, j, xr[S]);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (S == 0) quad_begin(j);
    write_src(smem + S * 64, src, B ? wb0 : wb1);        // table sigma + 4, other buffer
    src = sn;
    if constexpr (S == TPL - 1) {
      quad_end(j);
      __syncthreads();
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  for (int j = 0; j < nsteps; j += 2) {
    sub(I0{}, I0{}, j);
    sub(I0{}, I1{}, j);
    sub(I0{}, I2{}, j);
    sub(I0{}, I3{}, j);
    if (j + 1 >= nsteps) break;
    sub(I1{}, I0{}, j + 1);
    sub(I1{}, I1{}, j + 1);
    sub(I1{}, I2{}, j + 1);
    sub(I1{}, I3{}, j + 1);
  }
}

// Sub-step read addresses: rg's quarter at sub-step s, the lane's chunk and
// the buffer bit.
__device__ __forceinline__ unsigned read_mask(int g, int rg, int s, int b) {
  return (unsigned)((g << 4) | (((rg + s) & 3) << 6) | (b << 16));
}

// ----------------------------------------------------------------- grad_x
// MULTI: the workgroup's chunk may hold several quads (kq_chunk > 1), so the
// flush runs inside the loop; without it the one quad is flushed after the
// loop, which keeps the flush's registers out of the loop.
template <bool VEC, bool MULTI>
__global__ void __launch_bounds__(NT, 1)
custom_dx_kernel(const Params p) {
  __shared__ __align__(16) unsigned char smem[2 * QTAB];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane / 4, g = lane % 4;
  const int lb = logical_block();
  // A workgroup owns kq_chunk consecutive quads of taps of one row tile and
  // streams (quad, channel tile) steps through one table pipeline, so its
  // prologue is paid once per chunk, not once per quad.
  const int c = lb % p.kchunks;            // chunk of quads (consecutive blocks: same rows)
  const int tr = lb / p.kchunks;           // row tile
  const int j0 = c * p.kq_chunk;
  const int nsteps = MULTI ? min(p.kq_chunk, p.nq - j0) * p.tiles_o : p.tiles_o;
  const int r0 = tr * RT + wave * RPW + rg * RQ;
  const int xoff = (wave * RPW + rg * RQ) * 2;
  const int slot_bytes = p.Rpad * 2;
  const uint16_t* xtile = p.xt + (long long)tr * RT;

  float acc[TPL][RPL];
#pragma unroll
  for (int s = 0; s < TPL; ++s)
#pragma unroll
    for (int r = 0; r < RPL; ++r) acc[s][r] = 0.f;
  const __amdgpu_buffer_rsrc_t dyr = buffer_rsrc(p.dy, p.R * p.O * 4);
  DyRows<VEC> dro;
  dy_rows<VEC>(p, r0, 4 * g, dro);
  auto valid_of = [&](int t) { return min(4, max(0, p.O - CT * t - 4 * g)); };
  float dyv[RPL][4];
  load_dy<VEC>(dyr, dro, p.L, 0, valid_of(0), dyv);

  // step t = (quad j0 + t / tiles_o, channel tile t % tiles_o)
  auto col = [&](int t, int s, int og) {    // tap 4(j0 + t / tiles_o) + s
    const int q = MULTI ? t / p.tiles_o : 0, to = t - q * p.tiles_o;
    const int k = std::min(TPL * (j0 + q) + s, p.K - 1);
    return p.wt + (long long)k * p.Opad + CT * to + 4 * og;
  };
  // one quad per workgroup (!MULTI): one loop-invariant descriptor
  const __amdgpu_buffer_rsrc_t xs0 =
      buffer_rsrc(xtile + (long long)TPL * j0 * p.Rpad, TPL * slot_bytes);
  auto rows = [&](XRows& x, int t, int s) {
    if constexpr (MULTI) {
      const int q = t / p.tiles_o;
      load_x(x, buffer_rsrc(xtile + (long long)TPL * (j0 + q) * p.Rpad,
                            t < nsteps ? TPL * slot_bytes : 0),
             xoff, s * slot_bytes);
    } else {
      load_x(x, xs0, xoff, s * slot_bytes);
    }
  };
  // Reads of row quad h + 2 are issued before the FMAs of quad h, so at most
  // two quads of entries (32 registers) are in flight next to the 64
  // accumulators and 64 dy values.
  auto use = [&](auto bc, auto sc, int t, const XRows& x) __attribute__((always_inline)) {
    constexpr int B = decltype(bc)::value;
    constexpr int S = decltype(sc)::value;
    const unsigned gx = read_mask(g, rg, S, B);
    auto reads = [&](int h, float4 (&e)[RQ]) __attribute__((always_inline)) {
      const unsigned xd[2] = {x.v[h].x, x.v[h].y};
#pragma unroll
      for (int m = 0; m < RQ; ++m)
        e[m] = *(const float4*)(smem + (((xd[m >> 1] >> (16 * (m & 1))) & 0xffffu) ^ gx));
    };
    auto fmas = [&](int h, const float4 (&e)[RQ]) __attribute__((always_inline)) {
#pragma unroll
      for (int m = 0; m < RQ; ++m) {
        float a = acc[S][RQ * h + m];
        a = fmaf(dyv[RQ * h + m][0], e[m].x, a);
        a = fmaf(dyv[RQ * h + m][1], e[m].y, a);
        a = fmaf(dyv[RQ * h + m][2], e[m].z, a);
        a = fmaf(dyv[RQ * h + m][3], e[m].w, a);
        acc[S][RQ * h + m] = a;
      }
    };
    float4 e0[RQ], e1[RQ];
    reads(0, e0);
    reads(1, e1);
    __builtin_amdgcn_sched_barrier(0);
    fmas(0, e0);
    __builtin_amdgcn_sched_barrier(0);
    reads(2, e0);
    __builtin_amdgcn_sched_barrier(0);
    fmas(1, e1);
    __builtin_amdgcn_sched_barrier(0);
    reads(3, e1);
    __builtin_amdgcn_sched_barrier(0);
    fmas(2, e0);
    __builtin_amdgcn_sched_barrier(0);
    fmas(3, e1);
    // Pin the FMAs here: left free, the compiler sinks them past the next
    // sub-steps' loads and the epilogue, which drains the reads in flight.
#pragma unroll
    for (int r = 0; r < RPL; ++r) asm volatile("" : "+v"(acc[S][r]));
  };
  // The quad j's sums: over the row group's four chunk lanes, then lane g
  // stores slot g (tap 4j + ((rg + g) & 3)) for its 16 rows; the
  // accumulators restart at 0.
  auto flush = [&](int j) {
#pragma unroll
    for (int s = 0; s < TPL; ++s)
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        float a = acc[s][r];
        a += dpp<QP_XOR1>(a);
        a += dpp<QP_XOR2>(a);
        acc[s][r] = a;
      }
#pragma unroll
    for (int s = 0; s < TPL; ++s) {
      if (s != g) continue;
      const int k = TPL * j + ((rg + s) & 3);
      if (k >= p.K) continue;
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        const int rq = r0 + NRG * RQ * h;
        if (rq >= p.R) break;
        int n = rq / p.L, l = rq - n * p.L;
        if constexpr (VEC) {
          *(float4*)(p.out + ((long long)n * p.K + k) * p.L + l) =
              make_float4(acc[s][RQ * h], acc[s][RQ * h + 1], acc[s][RQ * h + 2],
                          acc[s][RQ * h + 3]);
        } else {
#pragma unroll
          for (int m = 0; m < RQ; ++m) {
            if (rq + m < p.R) p.out[((long long)n * p.K + k) * p.L + l] = acc[s][RQ * h + m];
            if (++l == p.L) { l = 0; ++n; }
          }
        }
      }
    }
#pragma unroll
    for (int s = 0; s < TPL; ++s)
#pragma unroll
      for (int r = 0; r < RPL; ++r) acc[s][r] = 0.f;
  };
  auto quad_end = [&](int t) {
    const int q = MULTI ? t / p.tiles_o : 0, to = t - q * p.tiles_o;
    if constexpr (MULTI)
      if (to == p.tiles_o - 1) flush(j0 + q);   // the quad's last channel tile
    // the next step's dy (its tables are already in the other buffer); an
    // unconditional load (the last step reloads tile 0), so the new values
    // can take the old registers
    const int tn = MULTI ? (to + 1 == p.tiles_o ? 0 : to + 1) : min(t + 1, p.tiles_o - 1);
    load_dy<VEC>(dyr, dro, p.L, CT * tn, valid_of(tn), dyv);
  };
  auto quad_begin = [&](int) {};
  table_stream(smem, p.tab, nsteps, col, rows, use, quad_end, quad_begin);
  if constexpr (!MULTI) flush(j0);
}

// ---------------------------------------- grad_w, tables rebuilt per row tile
// For L % 4 != 0 (rows of a quad straddle images, so dy is read one float at
// a time): a workgroup owns one 16-channel tile over 2048 rows, loads its dy
// once into registers and streams the tap quads through the table pipeline
// (split over several workgroups when the (row, channel) tile grid is smaller
// than the GPU, each writing its own taps' entries of the row tile's slice).
// The lane's partials are reduced over the 16 row groups of a wave with DPP
// row_shr, then over the waves through a two-stage LDS pipeline that needs no
// extra barrier, into one partial slice per row tile.
template <bool VEC>
__global__ void __launch_bounds__(NT, 1)
custom_dw_tile_kernel(const Params p) {
  __shared__ __align__(16) unsigned char smem[2 * QTAB];
  __shared__ float red1[2][RED1];          // [buf][wave][row q][g][tap][c]
  __shared__ float red2[2][RED2];          // [buf][wave][tap * 16 + o_local]
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane / 4, g = lane % 4;
  const int lb = logical_block();
  const int to = lb % p.tiles_o;           // channel tile (consecutive blocks: same rows)
  const int kc = (lb / p.tiles_o) % p.kchunks;   // chunk of tap quads
  const int tr = lb / p.tiles_o / p.kchunks;     // row tile
  const int j0 = kc * p.kq_chunk;          // the chunk's first quad
  const int nsteps = min(p.kq_chunk, p.nq - j0);
  const int r0 = tr * RT + wave * RPW + rg * RQ;
  const int xoff = (wave * RPW + rg * RQ) * 2;
  const int slot_bytes = p.Rpad * 2;
  const uint16_t* xtile = p.xt + (long long)tr * RT;
  float* slice = p.out + (long long)tr * p.O * p.K;

  float dyv[RPL][4];
  {
    DyRows<VEC> dro;
    dy_rows<VEC>(p, r0, 4 * g, dro);
    const int nvalid = min(4, max(0, p.O - CT * to - 4 * g));
    load_dy<VEC>(buffer_rsrc(p.dy, p.R * p.O * 4), dro, p.L, CT * to, nvalid, dyv);
    if (p.dys) {             // dy * factor[o], the product the caller would form
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float f = c < nvalid ? p.dys[CT * to + 4 * g + c] : 0.f;
#pragma unroll
        for (int r = 0; r < RPL; ++r) dyv[r][c] *= f;
      }
    }
  }
  float acc[TPL][4];

  // quads are counted from the chunk's first quad j0
  auto col = [&](int j, int s, int og) {   // quad j0 + j, tap 4(j0 + j) + s
    const int k = std::min(TPL * (j0 + j) + s, p.K - 1);
    return p.wt + (long long)k * p.Opad + CT * to + 4 * og;
  };
  auto rows = [&](XRows& x, int j, int s) {
    load_x(x, buffer_rsrc(xtile + (long long)TPL * (j0 + j) * p.Rpad,
                          j < nsteps ? TPL * slot_bytes : 0),
           xoff, s * slot_bytes);
  };
  auto use = [&](auto bc, auto sc, int, const XRows& x) __attribute__((always_inline)) {
    constexpr int B = decltype(bc)::value;
    constexpr int S = decltype(sc)::value;
    const unsigned gx = read_mask(g, rg, S, B);
    // all 16 reads in flight, then the FMAs in row order as they arrive
    float4 e[RPL];
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      const unsigned xd[2] = {x.v[h].x, x.v[h].y};
#pragma unroll
      for (int m = 0; m < RQ; ++m)
        e[RQ * h + m] =
            *(const float4*)(smem + (((xd[m >> 1] >> (16 * (m & 1))) & 0xffffu) ^ gx));
    }
    __builtin_amdgcn_sched_barrier(0);
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      a[0] = fmaf(dyv[r][0], e[r].x, a[0]);
      a[1] = fmaf(dyv[r][1], e[r].y, a[1]);
      a[2] = fmaf(dyv[r][2], e[r].z, a[2]);
      a[3] = fmaf(dyv[r][3], e[r].w, a[3]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      asm volatile("" : "+v"(a[c]));   // keep the FMAs in this sub-step (see grad_x)
      acc[S][c] = a[c];
    }
  };
  // Stage 1 (end of quad j): lane (rg, g) holds tap (rg + s) & 3 in slot s.
  // In a 16-lane DPP row the lanes of chunk g are rg = 4q..4q+3; lane
  // rg & 3 == 3 adds, for tap t, its own slot (t + 1) & 3 and the slots
  // (t + 2) & 3, (t + 3) & 3, t of the lanes 4, 8, 12 below it (the same tap)
  // and stores the row's sums.
  auto quad_end = [&](int j) {
    float out[TPL][4];
#pragma unroll
    for (int t = 0; t < TPL; ++t)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        out[t][c] = acc[(t + 1) & 3][c] + dpp<ROW_SHR4>(acc[(t + 2) & 3][c]) +
                    dpp<ROW_SHR8>(acc[(t + 3) & 3][c]) + dpp<ROW_SHR12>(acc[t][c]);
    if ((rg & 3) == 3) {
      float* d = &red1[j & 1][((wave * 4 + (rg >> 2)) * 4 + g) * 16];
#pragma unroll
      for (int t = 0; t < TPL; ++t)
        *(float4*)(d + 4 * t) = make_float4(out[t][0], out[t][1], out[t][2], out[t][3]);
    }
  };
  // Stage 2 (quad j + 1): thread (part w', output i) sums wave w''s four row
  // partials of output i = tap * 16 + o_local.  Stage 3 (quad j + 2): wave 0
  // sums the eight parts and stores the slice entry.
  auto stage2 = [&](int j) {
    const int i = tid & 63, w = tid >> 6;
    const int t = i >> 4, ol = i & 15;
    const float* s1 = &red1[j & 1][(w * 4 * 4 + (ol >> 2)) * 16 + 4 * t + (ol & 3)];
    red2[j & 1][w * 64 + i] = s1[0] + s1[4 * 16] + s1[8 * 16] + s1[12 * 16];
  };
  auto stage3 = [&](int j) {
    if (tid >= 64) return;
    const int t = tid >> 4, ol = tid & 15;
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) a += red2[j & 1][w * 64 + tid];
    const int k = TPL * (j0 + j) + t, o = CT * to + ol;
    if (k < p.K && o < p.O) slice[(long long)o * p.K + k] = a;
  };
  auto quad_begin = [&](int j) {
    if (j >= 1) stage2(j - 1);
    if (j >= 2) stage3(j - 2);
  };
  table_stream(smem, p.tab, nsteps, col, rows, use, quad_end, quad_begin);
  // drain the last two quads through stages 2 and 3
  if (nsteps >= 2) stage3(nsteps - 2);
  stage2(nsteps - 1);
  __syncthreads();
  stage3(nsteps - 1);
}

// ----------------------------------------------------------------- grad_w
// For L % 4 == 0.  grad_w contracts over the rows, so a workgroup keeps the
// tables of NB quads of taps resident for its whole run (NB = 2: eight taps,
// 128 KiB) and walks a chunk of row steps (NW waves x 256 rows each): a tap's
// 16 KiB table is built once per workgroup, not once per (row tile, tap), and
// the loop over the rows has no LDS writes and no barriers.  Workgroup
// (channel tile to, tap chunk kc = quads NB kc .. NB kc + NB - 1, row chunk
// rc = steps rc * rchunk ..).  Lane (rg, g) owns channels 4g..4g+3 of the
// tile and rows 256 wave + 64 h + 4 rg + m of every step; per row quad h it
// loads its rows' dy (four channels) and the rows' offsets in the quads' tap
// slots (lane g of a row group loads NB of the slots, DPP broadcasts share
// them), and accumulates acc[b][s][c] for tap 4(NB kc + b) + ((rg + s) & 3)
// (the operand's slot rotation, which keeps the reads conflict-free) over all
// its rows.  The loads of the next row quad are issued before the current one
// is summed; a wave skips row quads that lie wholly past R.  At the end the
// partials are combined over the row groups of a wave with DPP row_shr, then
// over the waves and row quads through LDS in a fixed order into the row
// chunk's slice [rchunks][O][K]; split_sum adds the slices in a fixed order.

// dy offsets of the lane's row quads (L % 4 == 0: a quad of rows never
// straddles two images, so its dy is one 16-byte load per channel), advanced
// one step of rows at a time without divisions: per quad h the byte offset
// of dy[n][o_lane][l] of its first row, l and the row.
struct DyWalk {
  unsigned off[NQ];
  int l[NQ];
  int r[NQ];
};

__device__ __forceinline__ void dy_walk_init(const Params& p, int r0, int o_lane, DyWalk& d) {
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    const int rq = r0 + NRG * RQ * h;
    const int n = rq / p.L, l = rq - n * p.L;
    d.r[h] = rq;
    d.l[h] = l;
    d.off[h] = (unsigned)((((long long)n * p.O + o_lane) * p.L + l) * 4);
  }
}

// A step of RS = q L + rem rows: step = 4 (q O L + rem), wrap = 4 (O L - L)
// when l passes L (unsigned arithmetic; the offsets stay below 2^32, checked
// on the host).
__device__ __forceinline__ void dy_walk_next(DyWalk& d, int h, int RS, int L, int rem,
                                             unsigned step, unsigned wrap) {
  const int l = d.l[h] + rem;
  const bool w = l >= L;             // selects, no branch
  d.r[h] += RS;
  d.l[h] = w ? l - L : l;
  d.off[h] = d.off[h] + step + (w ? wrap : 0u);
}

// dy of row quad h for the lane's four channels (ob = tile base): v[m][c].
// Valid offsets are below 2^31 (dy < 2 GiB); bit 31 set puts a load past the
// buffer, which returns 0 (arithmetic, not a branch: the loads stay
// unconditional).
__device__ __forceinline__ void load_dy_quad(__amdgpu_buffer_rsrc_t dyr, const DyWalk& d, int h,
                                             int R, int L, int ob, int valid,
                                             float (&v)[RQ][4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const unsigned bad = (unsigned)((c >= valid) | (d.r[h] >= R));
    const float4 f = __builtin_bit_cast(
        float4, __builtin_amdgcn_raw_buffer_load_b128(dyr, d.off[h] | (bad << 31),
                                                      (ob + c) * L * 4, 0));
    v[0][c] = f.x; v[1][c] = f.y; v[2][c] = f.z; v[3][c] = f.w;
  }
}

// DPP quad_perm broadcast of lane L of each group of four lanes.
template <int L>
__device__ __forceinline__ unsigned quad_bcast(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, L * 0x55, 0xf, 0xf, false);
}

template <int NB, int NW>
__global__ void __launch_bounds__(64 * NW, 1)
custom_dw_kernel(const Params p) {
  constexpr int RS = NW * RPW;                    // rows per step
  __shared__ __align__(16) unsigned char smem[NB * QTAB];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane / 4, g = lane % 4;
  const int lb = logical_block();
  const int to = lb % p.tiles_o;                  // channel tile (consecutive blocks: same rows)
  const int kc = (lb / p.tiles_o) % p.kchunks;    // tap chunk
  const int rc = lb / p.tiles_o / p.kchunks;      // row chunk
  const int j0 = kc * NB;                         // the chunk's first quad
  const int st0 = rc * p.rchunk, st1 = min(p.rsteps, st0 + p.rchunk);    // steps of RS rows
  const int slot_bytes = p.Rpad * 2;

  if (wave < 8) {  // the chunk's 4 NB tables, once, by eight waves
    const int og = __builtin_amdgcn_readfirstlane(wave % 4);
    const int hw = __builtin_amdgcn_readfirstlane(wave / 4);
    const int wb = (128 * hw + 2 * lane) * LINE + ((og ^ (lane & 3)) << 4);
    const __amdgpu_buffer_rsrc_t tabr = buffer_rsrc(p.tab, 256 * 256 * 4);
    unsigned w4[TPL * NB];
#pragma unroll
    for (int q = 0; q < TPL * NB; ++q) {
      const int k = min(TPL * j0 + q, p.K - 1);
      w4[q] = load_w4(p.wt + (long long)k * p.Opad + CT * to + 4 * og);
    }
    Src src[TPL * NB];
#pragma unroll
    for (int q = 0; q < TPL * NB; ++q) load_src(src[q], tabr, w4[q], lane, hw);
#pragma unroll
    for (int q = 0; q < TPL * NB; ++q)
      write_src(smem + (q / TPL) * QTAB + (q % TPL) * 64, src[q], wb);
  }

  const int nvalid = min(4, max(0, p.O - CT * to - 4 * g));
  float fac[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) fac[c] = p.dys && c < nvalid ? p.dys[CT * to + 4 * g + c] : 1.f;
  const __amdgpu_buffer_rsrc_t dyr = buffer_rsrc(p.dy, p.R * p.O * 4);
  // The chunk's 4 NB slots (fewer at the end of K) under one descriptor;
  // every part of a row-offset address is in the range-checked vector
  // offset, so rows past Rpad in the last slot read 0.  Lane g of a row
  // group loads slots NB g .. NB g + NB - 1 of its rows, and the group's four
  // lanes share them through DPP broadcasts.
  const __amdgpu_buffer_rsrc_t xall = buffer_rsrc(
      p.xt + (long long)TPL * j0 * p.Rpad, min(NB, p.nq - j0) * TPL * slot_bytes);
  unsigned xv[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
    xv[i] = (unsigned)((wave * RPW + rg * RQ) * 2) + (unsigned)(NB * g + i) * (unsigned)slot_bytes;
  DyWalk dw;
  dy_walk_init(p, st0 * RS + wave * RPW + rg * RQ, 4 * g, dw);
  const int qt = RS / p.L, rem = RS - qt * p.L;
  const unsigned step = 4u * ((unsigned)qt * (unsigned)p.O * (unsigned)p.L + (unsigned)rem);
  const unsigned wrap = 4u * ((unsigned)p.O * (unsigned)p.L - (unsigned)p.L);
  const int ob = CT * to;

  // loads of row quad h of the step whose rows start at byte tb of a slot
  auto load_quad = [&](int h, unsigned tb, uint2 (&xo)[NB][TPL], float (&dv)[RQ][4])
      __attribute__((always_inline)) {
    uint2 own[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
      own[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                             xall, xv[i] + tb + 2 * NRG * RQ * h, 0, 0));
    load_dy_quad(dyr, dw, h, p.R, p.L, ob, nvalid, dv);
    dy_walk_next(dw, h, RS, p.L, rem, step, wrap);
    auto put = [&](auto qc) __attribute__((always_inline)) {
      constexpr int q = decltype(qc)::value;
      xo[q / TPL][q % TPL] = make_uint2(quad_bcast<q / NB>(own[q % NB].x),
                                        quad_bcast<q / NB>(own[q % NB].y));
    };
    put(std::integral_constant<int, 0>{});
    put(std::integral_constant<int, 1>{});
    put(std::integral_constant<int, 2>{});
    put(std::integral_constant<int, 3>{});
    if constexpr (NB == 2) {
      put(std::integral_constant<int, 4>{});
      put(std::integral_constant<int, 5>{});
      put(std::integral_constant<int, 6>{});
      put(std::integral_constant<int, 7>{});
    }
  };

  float acc[NB][TPL][4];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int s = 0; s < TPL; ++s)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[b][s][c] = 0.f;

  // reads in batches of two slots (eight 16-byte reads in flight), each
  // followed by its FMAs
  // A wave whose rows of quad h all lie at or past R skips it (uniform: the
  // partial last step of a layer whose rows are not a multiple of the step).
  auto sum_quad = [&](const uint2 (&xo)[NB][TPL], const float (&dv0)[RQ][4], int st, int h)
      __attribute__((always_inline)) {
    if (st * RS + wave * RPW + NRG * RQ * h >= p.R) return;
    float dv[RQ][4];
#pragma unroll
    for (int m = 0; m < RQ; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) dv[m][c] = dv0[m][c] * fac[c];   // exact when fac = 1
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int sh = 0; sh < TPL; sh += 2) {
        float4 e[2][RQ];
#pragma unroll
        for (int s = sh; s < sh + 2; ++s) {
          const unsigned gx = read_mask(g, rg, s, b);
          const unsigned xd[2] = {xo[b][s].x, xo[b][s].y};
#pragma unroll
          for (int m = 0; m < RQ; ++m)
            e[s - sh][m] =
                *(const float4*)(smem + (((xd[m >> 1] >> (16 * (m & 1))) & 0xffffu) ^ gx));
        }
#pragma unroll
        for (int s = sh; s < sh + 2; ++s)
#pragma unroll
          for (int m = 0; m < RQ; ++m) {
            acc[b][s][0] = fmaf(dv[m][0], e[s - sh][m].x, acc[b][s][0]);
            acc[b][s][1] = fmaf(dv[m][1], e[s - sh][m].y, acc[b][s][1]);
            acc[b][s][2] = fmaf(dv[m][2], e[s - sh][m].z, acc[b][s][2]);
            acc[b][s][3] = fmaf(dv[m][3], e[s - sh][m].w, acc[b][s][3]);
          }
      }
  };

  __syncthreads();                                 // tables written
  uint2 xa[NB][TPL], xb[NB][TPL];
  float da[RQ][4], db[RQ][4];
  load_quad(0, (unsigned)(st0 * RS * 2), xa, da);
  for (int st = st0; st < st1; ++st) {
    const unsigned tb = (unsigned)(st * RS * 2);
    // quad h + 1 (the next step's quad 0 after quad 3) is requested before
    // quad h is summed; after the chunk's last step those loads are unused
    load_quad(1, tb, xb, db);
    sum_quad(xa, da, st, 0);
    load_quad(2, tb, xa, da);
    sum_quad(xb, db, st, 1);
    load_quad(3, tb, xb, db);
    sum_quad(xa, da, st, 2);
    load_quad(0, tb + RS * 2, xa, da);
    sum_quad(xb, db, st, 3);
  }

  __syncthreads();                                 // every wave is done with the tables
  // over the four row groups of a DPP row: lane rg & 3 == 3 adds, for tap t,
  // its slot (t + 1) & 3 and the slots (t + 2) & 3, (t + 3) & 3, t of the
  // lanes 4, 8, 12 below it (the same tap) and stores the row's sums
  float* red = (float*)smem;                       // [b][wave][row q][g][tap][c]
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
      float o4[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        o4[c] = acc[b][(t + 1) & 3][c] + dpp<ROW_SHR4>(acc[b][(t + 2) & 3][c]) +
                dpp<ROW_SHR8>(acc[b][(t + 3) & 3][c]) + dpp<ROW_SHR12>(acc[b][t][c]);
      if ((rg & 3) == 3)
        *(float4*)(red + (((b * NW + wave) * 4 + (rg >> 2)) * 4 + g) * 16 + 4 * t) =
            make_float4(o4[0], o4[1], o4[2], o4[3]);
    }
  }
  __syncthreads();
  if (tid < NB * 64) {                             // output (b, tap t, channel ol)
    const int b = tid >> 6, t = (tid >> 4) & 3, ol = tid & 15;
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        a += red[(((b * NW + w) * 4 + q) * 4 + (ol >> 2)) * 16 + 4 * t + (ol & 3)];
    const int k = TPL * (j0 + b) + t, o = CT * to + ol;
    if (k < p.K && o < p.O) p.out[((long long)rc * p.O + o) * p.K + k] = a;
  }
}

// ------------------------------------------------- fp32-class LUT GEMM
// y[n,o,l] = sum_k LUT[xi][wi] for a LUT whose entries are not all integers
// (csrc/claude/bgemm_lut_kernels.cuh:344-359 runs such LUTs through its
// tiled mainloop in fp32).  The sum is fp32 in ascending k, the reference's
// non-split order, so every output element is one chain of adds from 0.
// Tiles of 2048 rows x 16 channels use the pair-table stream above with the
// transposed fp32 LUT image as its source: lane (rg, g) adds channels
// 4g..4g+3 of its 16 rows, tap 4j + S at sub-step S of quad j (ascending),
// reading its row offsets from operand slot (S - rg) & 3, where the
// rotation put that tap.  All row groups read the same table quarter at a
// sub-step (the price of the ascending order: four-way LDS bank conflicts
// where the integer kernel has none).
struct F32Params {
  const uint16_t* xt; int Rpad;
  const uint8_t* wt; int Opad;
  const float* tab;        // transposed fp32 LUT: tab[w * 256 + x]
  int K, R, L, O, tiles_o, nq;
  int out_kind;            // ATX_OUT_F32 or ATX_OUT_DEQUANT
  const float* sx; const float* sw; const float* bias;
  float* y;                // [N][O][L]
};

template <bool VEC>
__global__ void __launch_bounds__(NT, 1)
lut_f32_kernel(const F32Params p) {
  __shared__ __align__(16) unsigned char smem[2 * QTAB];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane / 4, g = lane % 4;
  const int lb = logical_block();
  const int to = lb % p.tiles_o;           // channel tile (consecutive blocks: same rows)
  const int tr = lb / p.tiles_o;           // row tile
  const int r0 = tr * RT + wave * RPW + rg * RQ;
  const int slot_bytes = p.Rpad * 2;
  const int xoff = (wave * RPW + rg * RQ) * 2;
  const uint16_t* xtile = p.xt + (long long)tr * RT;

  float acc[RPL][4];
#pragma unroll
  for (int r = 0; r < RPL; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = 0.f;

  auto col = [&](int j, int s, int og) {   // quad j, tap 4j + s
    const int k = std::min(TPL * j + s, p.K - 1);
    return p.wt + (long long)k * p.Opad + CT * to + 4 * og;
  };
  auto rows = [&](XRows& x, int j, int s) {
    load_x(x, buffer_rsrc(xtile + (long long)TPL * j * p.Rpad, j < p.nq ? TPL * slot_bytes : 0),
           xoff + ((s - rg) & 3) * slot_bytes, 0);
  };
  auto use = [&](auto bc, auto sc, int j, const XRows& x) __attribute__((always_inline)) {
    constexpr int B = decltype(bc)::value;
    constexpr int S = decltype(sc)::value;
    if (TPL * j + S >= p.K) return;        // the last quad's taps past K
    const unsigned gx = (unsigned)((g << 4) | (S << 6) | (B << 16));
    float4 e[RPL];
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      const unsigned xd[2] = {x.v[h].x, x.v[h].y};
#pragma unroll
      for (int m = 0; m < RQ; ++m)
        e[RQ * h + m] =
            *(const float4*)(smem + (((xd[m >> 1] >> (16 * (m & 1))) & 0xffffu) ^ gx));
    }
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      acc[r][0] += e[r].x;
      acc[r][1] += e[r].y;
      acc[r][2] += e[r].z;
      acc[r][3] += e[r].w;
    }
#pragma unroll
    for (int r = 0; r < RPL; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(acc[r][c]));
  };
  auto none = [&](int) {};
  table_stream(smem, p.tab, p.nq, col, rows, use, none, none);

  // epilogue: channel o = 16 to + 4g + c, rows r0 + 64h + m
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int o = CT * to + 4 * g + c;
    if (o >= p.O) break;
    float sc = 0.f, b = 0.f;
    if (p.out_kind == ATX_OUT_DEQUANT) {
      sc = p.sx[0] * p.sw[o];
      if (p.bias) b = p.bias[o];
    }
    auto fin = [&](float a) {
      if (p.out_kind != ATX_OUT_DEQUANT) return a;
      const float t = a * sc;
      return p.bias ? b + t : t;
    };
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      const int rq = r0 + NRG * RQ * h;
      if (rq >= p.R) break;
      int n = rq / p.L, l = rq - n * p.L;
      if constexpr (VEC) {
        *(float4*)(p.y + ((long long)n * p.O + o) * p.L + l) =
            make_float4(fin(acc[RQ * h][c]), fin(acc[RQ * h + 1][c]), fin(acc[RQ * h + 2][c]),
                        fin(acc[RQ * h + 3][c]));
      } else {
#pragma unroll
        for (int m = 0; m < RQ; ++m) {
          if (rq + m < p.R) p.y[((long long)n * p.O + o) * p.L + l] = fin(acc[RQ * h + m][c]);
          if (++l == p.L) { l = 0; ++n; }
        }
      }
    }
  }
}

// Epilogue of an empty contraction (K = 0): every sum is 0.
__global__ void f32_empty_kernel(const F32Params p) {
  const long long numel = (long long)p.R * p.O;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < numel;
       i += (long long)gridDim.x * blockDim.x) {
    const int o = (int)((i / p.L) % p.O);
    float v = 0.f;
    if (p.out_kind == ATX_OUT_DEQUANT) {
      const float t = v * (p.sx[0] * p.sw[o]);
      v = p.bias ? p.bias[o] + t : t;
    }
    p.y[i] = v;
  }
}

// grad_x of a contraction over no channels.
__global__ void zero_fill_kernel(float* __restrict__ out, long long n) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    out[i] = 0.f;
}

}  // namespace cg
}  // namespace atx

using namespace atx;

static int custom_params(cg::Params& p, const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                         const float* dy, const float* tabT, int N, int K, int L, int O,
                         float* out, const char* who) {
  ATX_REQUIRE(N >= 0 && K >= 0 && L >= 0 && O >= 0, "%s: negative size", who);
  const long long R = (long long)N * L;
  ATX_REQUIRE(R <= 0x7fffffffLL - cg::RT, "%s: N*L too large", who);
  ATX_REQUIRE(Rpad >= R && Rpad % cg::RT == 0, "%s: bad Rpad %d", who, Rpad);
  if ((long long)Rpad > (1LL << 27))
    return set_error(ATX_ERANGE, "%s: Rpad %d exceeds 2^27 rows", who, Rpad);
  ATX_REQUIRE(Opad >= O && Opad % ATX_COL_TILE == 0, "%s: bad Opad %d", who, Opad);
  p = cg::Params{};
  p.xt = xt; p.Rpad = Rpad; p.wt = wt; p.Opad = Opad; p.tab = tabT; p.dy = dy; p.out = out;
  p.K = K; p.R = (int)R; p.L = L; p.O = O;
  if (R * O * 4 > 0x7fffffffLL)
    return set_error(ATX_ERANGE, "%s: dy of %lld x %d fp32 exceeds 2 GiB", who, R, O);
  p.tiles_r = (int)cdiv(R, cg::RT);
  p.tiles_o = (int)cdiv(O, cg::CT);
  p.nq = (int)cdiv(K, cg::TPL);
  p.kq_chunk = p.nq;
  p.kchunks = 1;
  return ATX_OK;
}

namespace atx {

int lut_gemm_f32_tiled(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                       const float* lutf32t, int N, int K, int L, int O, int out_kind,
                       const float* sx, const float* sw, const float* bias, float* y,
                       hipStream_t stream) {
  cg::F32Params p{};
  p.xt = xt; p.Rpad = Rpad; p.wt = wt; p.Opad = Opad; p.tab = lutf32t;
  p.K = K; p.R = N * L; p.L = L; p.O = O;
  p.tiles_o = (int)cdiv(O, cg::CT);
  p.nq = (int)cdiv(K, cg::TPL);
  p.out_kind = out_kind; p.sx = sx; p.sw = sw; p.bias = bias; p.y = y;
  const long long R = (long long)N * L;
  if (K == 0) {
    hipLaunchKernelGGL(cg::f32_empty_kernel, dim3(elem_grid(R * O, 256)), dim3(256), 0, stream,
                       p);
    return check_launch("f32_empty_kernel");
  }
  const long long blocks = cdiv(R, cg::RT) * p.tiles_o;
  ATX_REQUIRE(blocks < 0x7fffffffLL, "atx_lut_gemm: grid too large");
  if (L % 4 == 0)
    hipLaunchKernelGGL(cg::lut_f32_kernel<true>, dim3((unsigned)blocks), dim3(cg::NT), 0,
                       stream, p);
  else
    hipLaunchKernelGGL(cg::lut_f32_kernel<false>, dim3((unsigned)blocks), dim3(cg::NT), 0,
                       stream, p);
  return check_launch("lut_f32_kernel");
}

}  // namespace atx

extern "C" {

int atx_custom_grad_dx(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                       const float* dy, const float* tabT, int N, int K, int L, int O,
                       float* grad_x, hipStream_t stream) {
  cg::Params p;
  int rc = custom_params(p, xt, Rpad, wt, Opad, dy, tabT, N, K, L, O, grad_x,
                         "atx_custom_grad_dx");
  if (rc != ATX_OK) return rc;
  const long long numel = (long long)N * K * L;
  if (numel == 0) return ATX_OK;
  ATX_REQUIRE(grad_x, "atx_custom_grad_dx: null output");
  if (O == 0) {
    hipLaunchKernelGGL(cg::zero_fill_kernel, dim3(elem_grid(numel, 256)), dim3(256), 0, stream,
                       grad_x, numel);
    return check_launch("zero_fill_kernel");
  }
  ATX_REQUIRE(xt && wt && dy && tabT, "atx_custom_grad_dx: null operand");
  // quads per workgroup: enough (quad, channel tile) steps to amortize the
  // pipeline's prologue (at least 16), while keeping at least 1024
  // workgroups when there are that many quads to give out
  {
    const int want_steps = 16;
    int kq = (int)std::max<long long>(1, cdiv(want_steps, p.tiles_o));
    const long long min_blocks = 1024;
    while (kq > 1 && (long long)p.tiles_r * cdiv(p.nq, kq) < min_blocks) --kq;
    p.kq_chunk = std::min(kq, std::max(p.nq, 1));
    p.kchunks = (int)cdiv(p.nq, p.kq_chunk);
  }
  const long long blocks = (long long)p.tiles_r * p.kchunks;
  ATX_REQUIRE(blocks < 0x7fffffffLL, "atx_custom_grad_dx: grid too large");
  const bool multi = p.kq_chunk > 1;
  if (L % 4 == 0 && multi)
    hipLaunchKernelGGL((cg::custom_dx_kernel<true, true>), dim3((unsigned)blocks), dim3(cg::NT),
                       0, stream, p);
  else if (L % 4 == 0)
    hipLaunchKernelGGL((cg::custom_dx_kernel<true, false>), dim3((unsigned)blocks),
                       dim3(cg::NT), 0, stream, p);
  else if (multi)
    hipLaunchKernelGGL((cg::custom_dx_kernel<false, true>), dim3((unsigned)blocks),
                       dim3(cg::NT), 0, stream, p);
  else
    hipLaunchKernelGGL((cg::custom_dx_kernel<false, false>), dim3((unsigned)blocks),
                       dim3(cg::NT), 0, stream, p);
  return check_launch("custom_dx_kernel");
}

long long atx_custom_grad_dw_workspace_bytes(int N, int K, int L, int O) {
  if (N <= 0 || K <= 0 || L <= 0 || O <= 0) return 0;
  return cdiv((long long)N * L, cg::RT) * O * K * 4;
}

static int custom_dw_run(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                         const float* dy, const float* dy_scale, const float* tabT, int N,
                         int K, int L, int O, const uint8_t* mask_w, const float* scale_w,
                         const float* zsum, const float* zsx, const float* zzx, float* grad_w,
                         float* workspace, hipStream_t stream);

int atx_custom_grad_dw(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                       const float* dy, const float* dy_scale, const float* tabT, int N, int K,
                       int L, int O, const uint8_t* mask_w, const float* scale_w,
                       float* grad_w, float* workspace, hipStream_t stream) {
  return custom_dw_run(xt, Rpad, wt, Opad, dy, dy_scale, tabT, N, K, L, O, mask_w, scale_w,
                       nullptr, nullptr, nullptr, grad_w, workspace, stream);
}

int atx_custom_grad_dw_uint8(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                             const float* dy, const float* dy_scale, const float* tabT, int N,
                             int K, int L, int O, const uint8_t* mask_w, const float* scale_w,
                             const float* go_sum, const float* scale_x, const float* zero_x,
                             float* grad_w, float* workspace, hipStream_t stream) {
  ATX_REQUIRE((long long)O * K == 0 || (go_sum && scale_x && zero_x && scale_w),
              "atx_custom_grad_dw_uint8: null zero-point operand");
  return custom_dw_run(xt, Rpad, wt, Opad, dy, dy_scale, tabT, N, K, L, O, mask_w, scale_w,
                       go_sum, scale_x, zero_x, grad_w, workspace, stream);
}

static int custom_dw_run(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                         const float* dy, const float* dy_scale, const float* tabT, int N,
                         int K, int L, int O, const uint8_t* mask_w, const float* scale_w,
                         const float* zsum, const float* zsx, const float* zzx, float* grad_w,
                         float* workspace, hipStream_t stream) {
  cg::Params p;
  int rc = custom_params(p, xt, Rpad, wt, Opad, dy, tabT, N, K, L, O, workspace,
                         "atx_custom_grad_dw");
  if (rc != ATX_OK) return rc;
  p.dys = dy_scale;
  const long long numel = (long long)O * K;
  if (numel == 0) return ATX_OK;
  ATX_REQUIRE(grad_w && !(mask_w && !scale_w), "atx_custom_grad_dw: null output / scale");
  if (p.R == 0)
    return launch_split_sum(nullptr, 0, numel, K, mask_w, scale_w, grad_w, stream, zsum, zsx,
                            zzx);
  ATX_REQUIRE(xt && wt && dy && tabT && workspace, "atx_custom_grad_dw: null operand");
  if (L % 4 != 0 || (long long)Rpad * 16 > 0x7fffffffLL) {
    // Fewer (row, channel) tiles than CUs: split the tap quads over enough
    // workgroups to fill them (each workgroup writes its own taps' entries of
    // the row tile's slice, so no extra reduction).
    const long long tiles = (long long)p.tiles_r * p.tiles_o;
    if (tiles < 256 && p.nq >= 16) {
      const int want = (int)std::min<long long>(cdiv(256, tiles), p.nq / 8);
      p.kq_chunk = (int)cdiv(p.nq, want);
      p.kchunks = (int)cdiv(p.nq, p.kq_chunk);
    }
    const long long blocks = tiles * p.kchunks;
    ATX_REQUIRE(blocks < 0x7fffffffLL, "atx_custom_grad_dw: grid too large");
    hipLaunchKernelGGL(cg::custom_dw_tile_kernel<false>, dim3((unsigned)blocks), dim3(cg::NT),
                       0, stream, p);
    rc = check_launch("custom_dw_tile_kernel");
    if (rc != ATX_OK) return rc;
    return launch_split_sum(workspace, p.tiles_r, numel, K, mask_w, scale_w, grad_w, stream,
                            zsum, zsx, zzx);
  }
  // Workgroups of (channel tile, chunk of NB tap quads, chunk of row steps),
  // one per CU (128 KiB of tables), NW waves of 256 rows each.  Row chunks:
  // the fewest rounds of 256 workgroups x (steps per workgroup + the table
  // build, ~0.6 step), plus writing and summing one O x K slice per row chunk
  // (cost model in microseconds: 4.4 per 2048 rows x 16 channels x 8 taps).
  constexpr int NW = ATX_DW_WAVES;
  constexpr int RS = NW * 256;
  const int NB = p.nq >= 2 ? 2 : 1;
  ATX_REQUIRE((long long)(p.R + RS) * O * 4 <= 0xffffffffLL,
              "atx_custom_grad_dw: dy offsets exceed 32 bits");
  p.kq_chunk = NB;
  p.kchunks = (int)cdiv(p.nq, NB);
  p.rsteps = (int)cdiv(p.R, RS);
  const long long nw = (long long)p.tiles_o * p.kchunks;
  {
    double best = 0.0;
    int best_chunk = p.rsteps;
    for (int c = 1; c <= p.rsteps; ++c) {
      const int chunk = (int)cdiv(p.rsteps, c);
      if (c > 1 && chunk == (int)cdiv(p.rsteps, c - 1)) continue;
      const long long ce = cdiv(p.rsteps, chunk);
      const double rounds = (double)cdiv(nw * ce, 256);
      const double cost = rounds * (chunk * RS / 2048.0 + 0.6) * 4.4 * NB / 2 +
                          ce * (double)numel * 8 / 4e6;
      if (c == 1 || cost < best) { best = cost; best_chunk = chunk; }
    }
    p.rchunk = best_chunk;
  }
  const int slices = (int)cdiv(p.rsteps, p.rchunk);
  const long long blocks = nw * slices;
  ATX_REQUIRE(blocks < 0x7fffffffLL, "atx_custom_grad_dw: grid too large");
  if (NB == 2)
    hipLaunchKernelGGL((cg::custom_dw_kernel<2, NW>), dim3((unsigned)blocks), dim3(64 * NW), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((cg::custom_dw_kernel<1, NW>), dim3((unsigned)blocks), dim3(64 * NW), 0,
                       stream, p);
  rc = check_launch("custom_dw_kernel");
  if (rc != ATX_OK) return rc;
  return launch_split_sum(workspace, slices, numel, K, mask_w, scale_w, grad_w, stream, zsum,
                          zsx, zzx);
}

}  // extern "C"
