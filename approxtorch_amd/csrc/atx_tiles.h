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
// voff = byte offset of the lane's first quad within a slot).
__device__ __forceinline__ void load_x(XRows& x, __amdgpu_buffer_rsrc_t xs, int voff, int soff) {
#pragma unroll
  for (int h = 0; h < tiles::NQ; ++h)
    x.v[h] = __builtin_bit_cast(
        uint2, __builtin_amdgcn_raw_buffer_load_b64(xs, voff + 2 * tiles::NRG * tiles::RQ * h,
                                                    soff, 0));
}

}  // namespace atx
