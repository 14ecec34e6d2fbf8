// LDS throughput probe: the roofline denominator of the LUT GEMM (LDS bytes
// per clock per CU) and the bank structure its table layout relies on.
//
// Each workgroup fills 64 KiB of LDS (two workgroups fit on a CU, 16 waves).
// Every lane holds eight precomputed byte addresses; each iteration XORs
// them with a wave-uniform mask that moves whole rows, so the pattern's
// bank structure is the same in every iteration, and issues eight 16-byte
// accesses.  A read costs three VALU operations (address XOR and two
// three-input adds folding the data into one register), a write one, which
// keeps the VALU well below the LDS time even at 256 bytes per clock.
//   mode 0  read:  each 8-lane group reads one random 128-byte row
//   mode 1  read:  each wave reads 1 KiB contiguous (lane * 16)
//   mode 2  read:  as mode 0, with the row's parity equal to the group's
//   mode 3  read:  each 16-lane group reads one random 256-byte row
//   mode 4  read:  all lanes of a wave read the same random 128-byte row
//   mode 5  write: the table-build pattern: lane t writes 16 bytes at row
//                  2t + 128(u & 1), chunk position ((w + u/2) ^ t) & 7
//   mode 6  write: each wave writes 1 KiB contiguous (lane * 16)
//   mode 7  write: 8-byte accesses, each wave writes 512 B contiguous
//   mode 8  write: 4-byte accesses, each wave writes 256 B contiguous
//   mode 9  read:  each 4-lane group reads a random 64-byte row in quarter
//                  (group % 4) of a 256-byte line (quarters rotate by group)
//   mode 10 read:  as mode 9 with a random quarter per group
// The sum of everything read is stored so nothing is optimized away.
// Bytes moved per launch = blocks * 512 * iters * 8 * (16, or 8 / 4 for
// modes 7 / 8).

#include <hip/hip_runtime.h>

#include "../../include/atx_diag.h"

namespace atx_diag {

constexpr int PROBE_BYTES = 65536;

__device__ __forceinline__ unsigned mix(unsigned s) {
  s ^= s >> 16; s *= 0x7feb352du; s ^= s >> 15; s *= 0x846ca68bu; s ^= s >> 16;
  return s;
}

template <int MODE>
__global__ void __launch_bounds__(512) lds_probe_kernel(int iters, unsigned* out) {
  __shared__ __align__(16) unsigned char buf[PROBE_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < PROBE_BYTES / 4; i += blockDim.x)
    ((unsigned*)buf)[i] = (unsigned)i * 2654435761u;
  __syncthreads();

  const unsigned key = blockIdx.x * 4099u;
  const unsigned grp8 = (unsigned)(tid >> 3), grp16 = (unsigned)(tid >> 4);
  unsigned a[8];
  unsigned rowbits;          // address bits that select a row (moved by the mask)
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if constexpr (MODE == 0 || MODE == 2) {
      unsigned row = mix(key + grp8 * 977u + u * 7919u) & 511u;
      if (MODE == 2) row = (row & ~1u) | (grp8 & 1u);
      a[u] = row * 128u + (lane & 7) * 16u;
    } else if constexpr (MODE == 1 || MODE == 6) {
      a[u] = (mix(key + wave * 977u + u * 7919u) & 63u) * 1024u + lane * 16u;
    } else if constexpr (MODE == 9 || MODE == 10) {
      const unsigned grp4 = (unsigned)(tid >> 2);
      const unsigned h = mix(key + grp4 * 977u + u * 7919u);
      const unsigned quarter = MODE == 9 ? (grp4 & 3u) : ((h >> 9) & 3u);
      a[u] = (h & 255u) * 256u + quarter * 64u + (lane & 3) * 16u;
    } else if constexpr (MODE == 7 || MODE == 8) {
      a[u] = (mix(key + wave * 977u + u * 7919u) & 63u) * 1024u + lane * (MODE == 7 ? 8u : 4u);
    } else if constexpr (MODE == 3) {
      a[u] = (mix(key + grp16 * 977u + u * 7919u) & 255u) * 256u + (lane & 15) * 16u;
    } else if constexpr (MODE == 4) {
      a[u] = (mix(key + wave * 977u + u * 7919u) & 511u) * 128u + (lane & 7) * 16u;
    } else {
      a[u] = (2u * lane + 128u * (u & 1)) * 128u + ((((wave + (u >> 1)) ^ lane) & 7) << 4);
    }
  }
  if constexpr (MODE == 3 || MODE >= 9) rowbits = 0xff00u;
  else if constexpr (MODE == 1 || (MODE >= 6 && MODE <= 8)) rowbits = 0xfc00u;
  else if constexpr (MODE == 5) rowbits = 0x0100u;   // keeps rows 2t / 2t+1 pairs
  else rowbits = 0xff80u;

  unsigned acc = 0;
  for (int it = 0; it < iters; ++it) {
    const unsigned m = __builtin_amdgcn_readfirstlane(((unsigned)it * 0x9e3779b9u) & rowbits);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      unsigned char* p = buf + (a[u] ^ m);
      if constexpr (MODE <= 4 || MODE >= 9) {
        const uint4 v = *(const uint4*)p;
        acc += v.x + v.y;       // two three-input adds per read
        acc += v.z + v.w;
      } else if constexpr (MODE == 7) {
        *(uint2*)p = make_uint2(acc, (unsigned)it);
      } else if constexpr (MODE == 8) {
        *(unsigned*)p = acc + (unsigned)it;
      } else {
        *(uint4*)p = make_uint4(acc, (unsigned)it, (unsigned)u, 0u);
      }
    }
  }
  out[blockIdx.x * blockDim.x + tid] = acc;
}

// int32 add rate: 8 independent chains per lane, 64 v_add_u32 per iteration
// (inline asm so the adds are neither folded nor vectorized).
// VALU issue rate of one instruction form: 8 independent register chains
// per lane, 64 instructions per lane per iteration.
//   mode 0  v_add_u32                      (int32 add)
//   mode 1  v_add_u32_sdwa, sext WORD_1    (add of a dword's high signed half)
//   mode 2  v_add_u32_sdwa, sext WORD_0    (add of a dword's low signed half)
//   mode 3  v_bfe_i32                      (signed 16-bit field extract)
//   mode 4  v_pk_add_u16                   (two 16-bit adds)
//   mode 5  v_add3_u32                     (two int32 adds)
//   mode 6  v_perm_b32                     (byte permute)
//   mode 7  v_dot2_i32_i16                 (two 16x16 products + int32 add)
//   mode 8  v_add_u32 and v_add_u32_sdwa (sext WORD_1) alternating
//   mode 9  v_xor_b32
//   mode 10 v_ashrrev_i32
template <int MODE>
__device__ __forceinline__ void valu_op(unsigned& a, unsigned b) {
  if constexpr (MODE == 0) asm volatile("v_add_u32 %0, %0, %1" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 1)
    asm volatile("v_add_u32_sdwa %0, sext(%1), %0 dst_sel:DWORD dst_unused:UNUSED_PAD "
                 "src0_sel:WORD_1 src1_sel:DWORD" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 2)
    asm volatile("v_add_u32_sdwa %0, sext(%1), %0 dst_sel:DWORD dst_unused:UNUSED_PAD "
                 "src0_sel:WORD_0 src1_sel:DWORD" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 3) asm volatile("v_bfe_i32 %0, %1, 16, 16" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 4) asm volatile("v_pk_add_u16 %0, %0, %1" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 5) asm volatile("v_add3_u32 %0, %0, %1, %1" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 6) asm volatile("v_perm_b32 %0, %0, %1, %1" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 7) asm volatile("v_dot2_i32_i16 %0, %1, %1, %0" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 9) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 10) asm volatile("v_ashrrev_i32 %0, 16, %1" : "=v"(a) : "v"(b));
  else if constexpr (MODE == 11) asm volatile("v_and_b32 %0, 0xffff, %1" : "=v"(a) : "v"(b));
  else if constexpr (MODE == 12) asm volatile("v_lshrrev_b32 %0, 16, %1" : "=v"(a) : "v"(b));
  else if constexpr (MODE == 13) asm volatile("v_add_u32_e64 %0, %0, %1" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 14)
    asm volatile("v_bitop3_b32 %0, %0, %1, %1 bitop3:0x78" : "+v"(a) : "v"(b));
  else if constexpr (MODE == 15)
    asm volatile("v_xor_b32_sdwa %0, %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD "
                 "src0_sel:DWORD src1_sel:WORD_1" : "+v"(a) : "v"(b));
}

// 64-bit adds: v_lshl_add_u64 (one instruction) or the VCC carry pair
// v_add_co_u32 / v_addc_co_u32 (two).
template <int MODE>
__device__ __forceinline__ void valu_op64(unsigned long long& a, unsigned long long b) {
  if constexpr (MODE == 16) asm volatile("v_lshl_add_u64 %0, %1, 0, %0" : "+v"(a) : "v"(b));
  else {
    unsigned lo = (unsigned)a, hi = (unsigned)(a >> 32);
    asm volatile("v_add_co_u32_e32 %0, vcc, %2, %0\n\tv_addc_co_u32_e32 %1, vcc, %3, %1, vcc"
                 : "+v"(lo), "+v"(hi) : "v"((unsigned)b), "v"((unsigned)(b >> 32)) : "vcc");
    a = ((unsigned long long)hi << 32) | lo;
  }
}

// ONE_PER_CU: 96 KiB of LDS per workgroup, so one 512-thread workgroup runs
// per CU (two waves per SIMD, as in the LUT GEMM); otherwise several.
template <int MODE, bool ONE_PER_CU>
__global__ void __launch_bounds__(512) valu_probe_kernel(int iters, unsigned* out) {
  unsigned a[8], b[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    a[u] = threadIdx.x + u;
    b[u] = threadIdx.x * 7u + 3u * u + blockIdx.x;
  }
  if constexpr (MODE == 16 || MODE == 19) {
    unsigned long long a64[4], b64[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a64[u] = ((unsigned long long)a[2 * u + 1] << 32) | a[2 * u];
      b64[u] = ((unsigned long long)b[2 * u + 1] << 32) | b[2 * u];
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < 16; ++r)        // 64 adds: 64 (16) or 128 (19) instructions
#pragma unroll
        for (int u = 0; u < 4; ++u) valu_op64<MODE>(a64[u], b64[(u + r) & 3]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) { a[2 * u] = (unsigned)a64[u]; a[2 * u + 1] = (unsigned)(a64[u] >> 32); }
  } else {
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if constexpr (MODE == 8) {            // fast, slow, fast, slow, ...
            if (u & 1) valu_op<1>(a[u], b[(u + r) & 7]);
            else valu_op<0>(a[u], b[(u + r) & 7]);
          } else if constexpr (MODE == 17) {    // pairs: fast, fast, slow, slow, ...
            if (u & 2) valu_op<1>(a[u], b[(u + r) & 7]);
            else valu_op<0>(a[u], b[(u + r) & 7]);
          } else if constexpr (MODE == 18) {    // runs of eight fast, then eight slow
            if (r & 1) valu_op<1>(a[u], b[(u + r) & 7]);
            else valu_op<0>(a[u], b[(u + r) & 7]);
          } else {
            valu_op<MODE>(a[u], b[(u + r) & 7]);
          }
        }
    }
  }
  if constexpr (ONE_PER_CU) {
    __shared__ unsigned pad[24576];
    if (iters < 0) pad[threadIdx.x] = a[0];
    if (iters < 0) a[1] = pad[threadIdx.x ^ 1];
  }
  unsigned t = 0;
#pragma unroll
  for (int u = 0; u < 8; ++u) t += a[u];
  out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}


// ----------------------------------------------------------- inner-loop probe
// The LUT GEMM's main loop with its global loads taken out: 512 threads as 8
// waves (one workgroup per CU: 128 KiB of LDS), 128 int32 accumulators per
// lane, lane (row group rg = lane / 4, chunk g = lane % 4) reading its 16
// rows' 16-byte table chunks at row offset ^ (g*16 | quarter*64 |
// buffer*65536) with the quarter rotated per sub-step, and adding each chunk
// as the kernel does (one 32-bit add of the whole dword, one SDWA add of its
// high half).  The rows are pseudo-random per row group (the four lanes of a
// group share them, as in the kernel) and fixed over the run.  MODE bits:
// 1 LDS reads, 2 adds, 4 the table-build writes (two 16-byte stores per lane
// per sub-step, the kernel's pattern), 8 a barrier every four sub-steps.
// Without reads the adds take opaque register values; without adds the reads
// are consumed by empty asm.  A sub-step is 128 lookups per lane.
namespace inner {
constexpr int RPL = 16, NQ = 4, LINE = 256, QTAB = 65536;

template <int S, int B>
__device__ __forceinline__ unsigned quarter_mask(unsigned base) {
  unsigned t;
  asm volatile("v_add_u32 %0, %1, %2\n\tv_and_b32 %0, %3, %0\n\tv_or_b32 %0, %4, %0"
               : "=&v"(t) : "n"(S << 6), "v"(base), "n"(0xf0), "n"(B << 16));
  return t;
}

template <bool GROUPED>
__device__ __forceinline__ void add8(int (&a)[8], const uint4 e) {
  if constexpr (GROUPED) {
    // the four whole-dword adds adjacent, then the four SDWA adds
    asm("v_add_u32_e32 %0, %4, %0\n\tv_add_u32_e32 %1, %5, %1\n\t"
        "v_add_u32_e32 %2, %6, %2\n\tv_add_u32_e32 %3, %7, %3"
        : "+v"(a[0]), "+v"(a[2]), "+v"(a[4]), "+v"(a[6])
        : "v"(e.x), "v"(e.y), "v"(e.z), "v"(e.w));
    asm("v_add_u32_sdwa %0, sext(%4), %0 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD\n\t"
        "v_add_u32_sdwa %1, sext(%5), %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD\n\t"
        "v_add_u32_sdwa %2, sext(%6), %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD\n\t"
        "v_add_u32_sdwa %3, sext(%7), %3 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD"
        : "+v"(a[1]), "+v"(a[3]), "+v"(a[5]), "+v"(a[7])
        : "v"(e.x), "v"(e.y), "v"(e.z), "v"(e.w));
  } else {
    const unsigned d[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] = (int)((unsigned)a[2 * i] + d[i]);
      a[2 * i + 1] += ((int)d[i]) >> 16;
    }
  }
}

template <int MODE>
__device__ __forceinline__ void sub(int (&acc)[RPL][8], unsigned char* smem,
                                    const unsigned (&xd)[8], unsigned gx, int wb, uint4 wv,
                                    uint4 (&fk)[8]) {
#pragma unroll
  for (int hh = 0; hh < NQ; hh += 2) {
    uint4 e[8];
    if constexpr (MODE & 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned x = xd[hh * 2 + j];
        e[2 * j] = *(const uint4*)(smem + ((x & 0xffffu) ^ gx));
        e[2 * j + 1] = *(const uint4*)(smem + ((x >> 16) ^ gx));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        asm volatile("" : "+v"(fk[j].x), "+v"(fk[j].y), "+v"(fk[j].z), "+v"(fk[j].w));
        e[j] = fk[j];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (MODE & 2) add8<(MODE & 16) != 0>(acc[4 * hh + j], e[j]);
      else asm volatile("" :: "v"(e[j].x), "v"(e[j].y), "v"(e[j].z), "v"(e[j].w));
    }
  }
  if constexpr (MODE & 2) {
#pragma unroll
    for (int jj = 0; jj < RPL; ++jj)
#pragma unroll
      for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(acc[jj][e]));
  }
  if constexpr (MODE & 4) {
    *(uint4*)(smem + wb) = wv;
    *(uint4*)(smem + wb + LINE) = wv;
  }
}

template <int MODE>
__global__ void __launch_bounds__(512, 1) inner_probe_kernel(int iters, unsigned* out) {
  __shared__ __align__(16) unsigned char smem[2 * QTAB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = lane / 4, g = lane % 4;
  for (int i = tid; i < 2 * QTAB / 4; i += 512) ((unsigned*)smem)[i] = i * 2654435761u;
  __syncthreads();
  unsigned xd[8];
  const unsigned grp = blockIdx.x * 128u + (unsigned)(tid >> 2);   // row group
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const unsigned r0 = mix(grp * 977u + 2u * i) & 255u, r1 = mix(grp * 977u + 2u * i + 1u) & 255u;
    const unsigned o0 = r0 * 256 + ((r0 >> 1) & 3) * 16, o1 = r1 * 256 + ((r1 >> 1) & 3) * 16;
    xd[i] = o0 | (o1 << 16);
  }
  const unsigned gbase = (unsigned)((rg << 6) | (g << 4));
  const int og = wave % 4, hw = wave / 4;
  const int wb0 = (128 * hw + 2 * lane) * LINE + ((og ^ (lane & 3)) << 4);
  int acc[RPL][8];
#pragma unroll
  for (int j = 0; j < RPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0;
  uint4 wv = make_uint4(tid, tid + 1, tid + 2, tid + 3);
  uint4 fk[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) fk[j] = make_uint4(xd[j], xd[j] + 1, xd[j] * 3, xd[j] ^ 5);
  for (int it = 0; it < iters; ++it) {      // eight sub-steps (two quads) per iteration
    sub<MODE>(acc, smem, xd, quarter_mask<0, 0>(gbase), wb0 + QTAB, wv, fk);
    sub<MODE>(acc, smem, xd, quarter_mask<1, 0>(gbase), wb0 + QTAB + 64, wv, fk);
    sub<MODE>(acc, smem, xd, quarter_mask<2, 0>(gbase), wb0 + QTAB + 128, wv, fk);
    sub<MODE>(acc, smem, xd, quarter_mask<3, 0>(gbase), wb0 + QTAB + 192, wv, fk);
    if constexpr (MODE & 8) __syncthreads();
    sub<MODE>(acc, smem, xd, quarter_mask<0, 1>(gbase), wb0, wv, fk);
    sub<MODE>(acc, smem, xd, quarter_mask<1, 1>(gbase), wb0 + 64, wv, fk);
    sub<MODE>(acc, smem, xd, quarter_mask<2, 1>(gbase), wb0 + 128, wv, fk);
    sub<MODE>(acc, smem, xd, quarter_mask<3, 1>(gbase), wb0 + 192, wv, fk);
    if constexpr (MODE & 8) __syncthreads();
    wv.x += 1;
  }
  int t = 0;
#pragma unroll
  for (int j = 0; j < RPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) t += acc[j][e];
  out[blockIdx.x * 512 + tid] = (unsigned)t;
}

// SWAR accumulation (bit 32 of the mode): a 16-byte table chunk holds six
// channels in four dwords, each dword a 16-bit entry in bits 0-19 plus one
// byte of a third channel in bits 20-31 (dword 2m+1 holds that channel's
// high byte).  Four plain 32-bit adds per chunk; sixteen k-steps fit the
// fields, then a flush moves them into int32 sums.  Lookups per sub-step:
// 16 rows x 6 channels per lane.
template <int MODE>
__global__ void __launch_bounds__(512, 1) swar_probe_kernel(int iters, unsigned* out) {
  __shared__ __align__(16) unsigned char smem[2 * QTAB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = lane / 4, g = lane % 4;
  for (int i = tid; i < 2 * QTAB / 4; i += 512) ((unsigned*)smem)[i] = (i * 2654435761u) & 0x0ff0ffffu;
  __syncthreads();
  unsigned xd[8];
  const unsigned grp = blockIdx.x * 128u + (unsigned)(tid >> 2);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const unsigned r0 = mix(grp * 977u + 2u * i) & 255u, r1 = mix(grp * 977u + 2u * i + 1u) & 255u;
    const unsigned o0 = r0 * 256 + ((r0 >> 1) & 3) * 16, o1 = r1 * 256 + ((r1 >> 1) & 3) * 16;
    xd[i] = o0 | (o1 << 16);
  }
  const unsigned gbase = (unsigned)((rg << 6) | (g << 4));
  const int og = wave % 4, hw = wave / 4;
  const int wb0 = (128 * hw + 2 * lane) * LINE + ((og ^ (lane & 3)) << 4);
  unsigned sw[RPL][4];        // SWAR fields
  int wide[RPL][6];           // int32 sums
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
#pragma unroll
    for (int c = 0; c < 4; ++c) sw[j][c] = 0;
#pragma unroll
    for (int c = 0; c < 6; ++c) wide[j][c] = 0;
  }
  uint4 wv = make_uint4(tid, tid + 1, tid + 2, tid + 3);
  auto sub = [&](unsigned gx, int wb) __attribute__((always_inline)) {
#pragma unroll
    for (int hh = 0; hh < NQ; hh += 2) {    // two batches of eight reads
      uint4 e[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const unsigned x0 = xd[2 * (hh + h)], x1 = xd[2 * (hh + h) + 1];
        e[4 * h] = *(const uint4*)(smem + ((x0 & 0xffffu) ^ gx));
        e[4 * h + 1] = *(const uint4*)(smem + ((x0 >> 16) ^ gx));
        e[4 * h + 2] = *(const uint4*)(smem + ((x1 & 0xffffu) ^ gx));
        e[4 * h + 3] = *(const uint4*)(smem + ((x1 >> 16) ^ gx));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        unsigned* a = sw[4 * hh + j];
        a[0] += e[j].x; a[1] += e[j].y; a[2] += e[j].z; a[3] += e[j].w;
      }
    }
#pragma unroll
    for (int j = 0; j < RPL; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(sw[j][c]));
    if constexpr (MODE & 4) {
      *(uint4*)(smem + wb) = wv;
      *(uint4*)(smem + wb + LINE) = wv;
    }
  };
  auto flush = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const unsigned d0 = sw[j][2 * m], d1 = sw[j][2 * m + 1];
        wide[j][3 * m] += (int)(d0 & 0xfffffu);
        wide[j][3 * m + 1] += (int)(d1 & 0xfffffu);
        wide[j][3 * m + 2] += (int)((d0 >> 20) + ((d1 >> 20) << 8));
        sw[j][2 * m] = 0; sw[j][2 * m + 1] = 0;
      }
    }
  };
  for (int it = 0; it < iters; ++it) {      // eight sub-steps per iteration
    sub(atx_diag::inner::quarter_mask<0, 0>(gbase), wb0 + QTAB);
    sub(atx_diag::inner::quarter_mask<1, 0>(gbase), wb0 + QTAB + 64);
    sub(atx_diag::inner::quarter_mask<2, 0>(gbase), wb0 + QTAB + 128);
    sub(atx_diag::inner::quarter_mask<3, 0>(gbase), wb0 + QTAB + 192);
    if constexpr (MODE & 8) __syncthreads();
    sub(atx_diag::inner::quarter_mask<0, 1>(gbase), wb0);
    sub(atx_diag::inner::quarter_mask<1, 1>(gbase), wb0 + 64);
    sub(atx_diag::inner::quarter_mask<2, 1>(gbase), wb0 + 128);
    sub(atx_diag::inner::quarter_mask<3, 1>(gbase), wb0 + 192);
    if constexpr (MODE & 8) __syncthreads();
    if (it & 1) flush();                   // every sixteen k-steps
    wv.x += 1;
  }
  int t = 0;
#pragma unroll
  for (int j = 0; j < RPL; ++j)
#pragma unroll
    for (int c = 0; c < 6; ++c) t += wide[j][c];
  out[blockIdx.x * 512 + tid] = (unsigned)t;
}
}  // namespace inner
}  // namespace atx_diag

using namespace atx_diag;

template <int MODE>
static void valu_launch(bool one, int blocks, int iters, unsigned* out, hipStream_t stream) {
  if (one)
    hipLaunchKernelGGL((valu_probe_kernel<MODE, true>), dim3(blocks), dim3(512), 0, stream, iters, out);
  else
    hipLaunchKernelGGL((valu_probe_kernel<MODE, false>), dim3(blocks), dim3(512), 0, stream, iters, out);
}


extern "C" {

int atx_lds_probe(int mode, int blocks, int iters, unsigned* out, hipStream_t stream) {
  if (!(mode >= 0 && mode <= 10 && blocks > 0 && iters > 0 && out)) return (int)hipErrorInvalidValue;
  switch (mode) {
    case 0: hipLaunchKernelGGL(lds_probe_kernel<0>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 1: hipLaunchKernelGGL(lds_probe_kernel<1>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 2: hipLaunchKernelGGL(lds_probe_kernel<2>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 3: hipLaunchKernelGGL(lds_probe_kernel<3>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 4: hipLaunchKernelGGL(lds_probe_kernel<4>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 5: hipLaunchKernelGGL(lds_probe_kernel<5>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 6: hipLaunchKernelGGL(lds_probe_kernel<6>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 7: hipLaunchKernelGGL(lds_probe_kernel<7>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 8: hipLaunchKernelGGL(lds_probe_kernel<8>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 9: hipLaunchKernelGGL(lds_probe_kernel<9>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    default: hipLaunchKernelGGL(lds_probe_kernel<10>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
  }
  return (int)hipGetLastError();
}

int atx_valu_probe(int mode, int blocks, int iters, unsigned* out, hipStream_t stream) {
  const bool one = (mode & 0x100) != 0;
  mode &= 0xff;
  if (!(mode >= 0 && mode <= 19 && blocks > 0 && iters > 0 && out)) return (int)hipErrorInvalidValue;
  switch (mode) {
    case 0: valu_launch<0>(one, blocks, iters, out, stream); break;
    case 1: valu_launch<1>(one, blocks, iters, out, stream); break;
    case 2: valu_launch<2>(one, blocks, iters, out, stream); break;
    case 3: valu_launch<3>(one, blocks, iters, out, stream); break;
    case 4: valu_launch<4>(one, blocks, iters, out, stream); break;
    case 5: valu_launch<5>(one, blocks, iters, out, stream); break;
    case 6: valu_launch<6>(one, blocks, iters, out, stream); break;
    case 7: valu_launch<7>(one, blocks, iters, out, stream); break;
    case 8: valu_launch<8>(one, blocks, iters, out, stream); break;
    case 9: valu_launch<9>(one, blocks, iters, out, stream); break;
    case 10: valu_launch<10>(one, blocks, iters, out, stream); break;
    case 11: valu_launch<11>(one, blocks, iters, out, stream); break;
    case 12: valu_launch<12>(one, blocks, iters, out, stream); break;
    case 13: valu_launch<13>(one, blocks, iters, out, stream); break;
    case 14: valu_launch<14>(one, blocks, iters, out, stream); break;
    case 15: valu_launch<15>(one, blocks, iters, out, stream); break;
    case 16: valu_launch<16>(one, blocks, iters, out, stream); break;
    case 17: valu_launch<17>(one, blocks, iters, out, stream); break;
    case 18: valu_launch<18>(one, blocks, iters, out, stream); break;
    default: valu_launch<19>(one, blocks, iters, out, stream); break;
  }
  return (int)hipGetLastError();
}

int atx_inner_probe(int mode, int blocks, int iters, unsigned* out, hipStream_t stream) {
  if (!(blocks > 0 && iters > 0 && out)) return (int)hipErrorInvalidValue;
  switch (mode) {
    case 1: hipLaunchKernelGGL(inner::inner_probe_kernel<1>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 2: hipLaunchKernelGGL(inner::inner_probe_kernel<2>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 3: hipLaunchKernelGGL(inner::inner_probe_kernel<3>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 4: hipLaunchKernelGGL(inner::inner_probe_kernel<4>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 7: hipLaunchKernelGGL(inner::inner_probe_kernel<7>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 11: hipLaunchKernelGGL(inner::inner_probe_kernel<11>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 15: hipLaunchKernelGGL(inner::inner_probe_kernel<15>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 18: hipLaunchKernelGGL(inner::inner_probe_kernel<18>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 19: hipLaunchKernelGGL(inner::inner_probe_kernel<19>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 31: hipLaunchKernelGGL(inner::inner_probe_kernel<31>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 35: hipLaunchKernelGGL(inner::swar_probe_kernel<3>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 47: hipLaunchKernelGGL(inner::swar_probe_kernel<15>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

}  // extern "C"
