// LDS throughput probe: measures the roofline denominator of the LUT GEMM
// (LDS bytes per clock per CU) and the bank structure its layout relies on.
// Each workgroup fills 64 KiB of LDS; every lane issues `iters` x 8 reads.
// Addresses come from a per-group hash (no cross-lane operations, which
// would themselves use the LDS pipe):
//   mode 0  ds_read_b128, each 8-lane group reads one random 128-byte row
//   mode 1  ds_read_b128, each wave reads 1 KiB contiguous
//   mode 2  as mode 0, but the row's parity equals the 8-lane group's parity
//   mode 3  ds_read_b128, each 16-lane group reads one random 256-byte row
//   mode 4  ds_read_u16 at independent random addresses (a plain LUT gather)
//   mode 5  ds_write_b32, each 32-lane half-wave writes one random 128-byte row
// The sum of what was read is stored so nothing is optimized away.

#include "atx_internal.h"

namespace atx {

constexpr int PROBE_BYTES = 65536;

__device__ __forceinline__ unsigned mix(unsigned s) {
  s ^= s >> 16; s *= 0x7feb352du; s ^= s >> 15; s *= 0x846ca68bu; s ^= s >> 16;
  return s;
}

template <int MODE>
__global__ void __launch_bounds__(512) lds_probe_kernel(int iters, unsigned* out) {
  __shared__ __align__(16) unsigned char buf[PROBE_BYTES];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < PROBE_BYTES / 4; i += blockDim.x)
    ((unsigned*)buf)[i] = (unsigned)i * 2654435761u;
  __syncthreads();
  const unsigned grp8 = (unsigned)(tid >> 3), grp16 = (unsigned)(tid >> 4);
  const unsigned key = blockIdx.x * 4099u;
  unsigned acc = 0;
  for (int it = 0; it < iters; ++it) {
    // one hash per 8 reads; read u derives its address with a multiply-add
    const unsigned h8 = mix(key + grp8 * 977u + (unsigned)it * 131071u);
    const unsigned h16 = mix(key + grp16 * 977u + (unsigned)it * 131071u);
    const unsigned hw = mix(key + (unsigned)(tid >> 6) * 977u + (unsigned)it * 131071u);
    const unsigned hl = mix(key + (unsigned)tid * 977u + (unsigned)it * 131071u);
    const unsigned hh = mix(key + (unsigned)(tid >> 5) * 977u + (unsigned)it * 131071u);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const unsigned step = (unsigned)it * 8u + u;
      const unsigned mul = 2u * u + 1u, add = (unsigned)u * 0x9e3779b9u;
      if constexpr (MODE == 0 || MODE == 2) {
        unsigned row = (h8 * mul + add) >> 23;
        if (MODE == 2) row = (row & ~1u) | (grp8 & 1u);
        const uint4 v = *(const uint4*)(buf + row * 128u + (lane & 7) * 16u);
        acc += v.x ^ v.y ^ v.z ^ v.w;
      } else if constexpr (MODE == 1) {
        const unsigned base = ((hw * mul + add) >> 26) * 1024u;
        const uint4 v = *(const uint4*)(buf + base + lane * 16u);
        acc += v.x ^ v.y ^ v.z ^ v.w;
      } else if constexpr (MODE == 3) {
        const unsigned row = (h16 * mul + add) >> 24;
        const uint4 v = *(const uint4*)(buf + row * 256u + (lane & 15) * 16u);
        acc += v.x ^ v.y ^ v.z ^ v.w;
      } else if constexpr (MODE == 4) {
        const unsigned a = ((hl * mul + add) >> 16) & 0xfffeu;
        acc += *(const unsigned short*)(buf + a);
      } else {
        const unsigned row = (hh * mul + add) >> 23;
        *(unsigned*)(buf + row * 128u + (lane & 31) * 4u) = step;
      }
    }
  }
  out[blockIdx.x * blockDim.x + tid] = acc;
}

}  // namespace atx

using namespace atx;

extern "C" {

// Launches `blocks` x 512 threads of the probe; the caller times it (events
// on `stream`).  Bytes moved = blocks * 512 * iters * 8 * {16,16,16,16,2,4}[mode].
int atx_lds_probe(int mode, int blocks, int iters, unsigned* out, hipStream_t stream) {
  ATX_REQUIRE(mode >= 0 && mode <= 5 && blocks > 0 && iters > 0 && out,
              "atx_lds_probe: bad arguments");
  switch (mode) {
    case 0: hipLaunchKernelGGL(lds_probe_kernel<0>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 1: hipLaunchKernelGGL(lds_probe_kernel<1>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 2: hipLaunchKernelGGL(lds_probe_kernel<2>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 3: hipLaunchKernelGGL(lds_probe_kernel<3>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    case 4: hipLaunchKernelGGL(lds_probe_kernel<4>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
    default: hipLaunchKernelGGL(lds_probe_kernel<5>, dim3(blocks), dim3(512), 0, stream, iters, out); break;
  }
  return check_launch("lds_probe_kernel");
}

}  // extern "C"
