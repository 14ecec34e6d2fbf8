// Device helpers shared by the LDS-table kernels (the LUT GEMM forward and
// the pair-table gradients): both tile 2048 rows over 8 waves, lane
// (row group rg = lane / 4, chunk g = lane % 4) owning rows
// 256 wave + 64 h + 4 rg + m (h, m = 0..3), and read the row-offset operand
// [Kpad][Rpad] written by the pack / im2col kernels.
#pragma once

#include "atx_internal.h"

namespace atx {
namespace tiles {

constexpr int NRG = 16;            // row groups per wave
constexpr int RQ = 4;              // consecutive rows per lane quad
constexpr int NQ = 4;              // quads per lane (stride NRG * RQ rows)
constexpr int RPL = RQ * NQ;       // rows per lane (16)
constexpr int RPW = NRG * RPL;     // rows per wave (256)

}  // namespace tiles

// Blocks are dispatched round-robin over the 8 XCDs (bid % 8).  Gives each
// XCD a contiguous range of logical blocks, so consecutive logical blocks
// (which share operand tiles) share that XCD's L2.
__device__ __forceinline__ int logical_block() {
  const int bid = blockIdx.x, nb = gridDim.x;
  const int q = nb >> 3, rem = nb & 7;
  const int xcd = bid & 7, slot = bid >> 3;
  return xcd < rem ? xcd * (q + 1) + slot : rem * (q + 1) + (xcd - rem) * q + slot;
}

// Raw buffer descriptor (word 3 of the gfx9-family descriptor: 32-bit
// elements, no swizzle) over `bytes` bytes at a wave-uniform base.  Buffer
// loads take the per-step offsets in scalar registers, so they cost no
// per-lane 64-bit address arithmetic; accesses at or beyond `bytes` return 0
// without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes,
                                           0x00020000);
}

// Row offsets of the lane's quads: v[h] = rows NRG*RQ*h + 4rg + 0..3, two per
// dword.
struct XRows { uint2 v[tiles::NQ]; };

// Row offsets of the lane's quads from slot soff / (2 Rpad) of a quad's
// row-offset block (xs = descriptor over the quad's four slots of the tile,
// voff = byte offset of the lane's first quad within a slot).  The quads'
// 128-byte steps go into the scalar offset, so all four loads share the one
// per-lane offset register.
__device__ __forceinline__ void load_x(XRows& x, __amdgpu_buffer_rsrc_t xs, int voff, int soff) {
#pragma unroll
  for (int h = 0; h < tiles::NQ; ++h)
    x.v[h] = __builtin_bit_cast(
        uint2, __builtin_amdgcn_raw_buffer_load_b64(xs, voff,
                                                    soff + 2 * tiles::NRG * tiles::RQ * h, 0));
}

// Read XOR mask of sub-step S from quad buffer B for a lane with
// base = (rg << 6) | (g << 4): chunk g in bits 4-5, table quarter
// (rg + S) & 3 in bits 6-7, the buffer in bit 16.  Formed in place by asm
// the compiler can neither hoist (four masks kept live across a kernel's
// main loop cost registers that then spill) nor fold into every address.
template <int S, int B>
__device__ __forceinline__ unsigned quarter_mask(unsigned base) {
  unsigned t;
  asm volatile("v_add_u32 %0, %1, %2\n\tv_and_b32 %0, %3, %0\n\tv_or_b32 %0, %4, %0"
               : "=&v"(t) : "n"(S << 6), "v"(base), "n"(0xf0), "n"(B << 16));
  return t;
}

}  // namespace atx
