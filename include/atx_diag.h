/*
 * atx_diag.h — measurement probes of libatx_diag.so (not part of libatx.so).
 *
 * These kernels have no counterpart in the reference: they measure the
 * hardware ceilings the LUT GEMM is reported against (LDS bytes per clock for
 * the access patterns its tables use, and the int32 VALU add rate).  Only
 * bench.py --probe-lds loads this library.  Return value: a hipError_t code
 * (0 = success).
 */
#ifndef ATX_DIAG_H
#define ATX_DIAG_H

#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

/* LDS throughput: blocks x 512 threads, each lane issuing iters*8 accesses
 * of pattern `mode`:
 *   0 read, one random 128-byte row per 8-lane group;
 *   1 read, 1 KiB contiguous per wave;
 *   2 read, as 0 with the row parity equal to the group parity;
 *   3 read, one random 256-byte row per 16-lane group;
 *   4 read, one random 128-byte row per wave (broadcast);
 *   5 write, the LUT GEMM table-build pattern;
 *   6 write, 1 KiB contiguous per wave;
 *   7 write, 8-byte accesses, 512 B contiguous per wave;
 *   8 write, 4-byte accesses, 256 B contiguous per wave;
 *   9 read, one random 64-byte row per 4-lane group, in quarter (group % 4)
 *     of a 256-byte line;
 *  10 read, as 9 with a random quarter.
 * Bytes moved = blocks * 512 * iters * 8 * {16, 8, 4} (modes 0-6 and 9-10,
 * 7, 8).  out: blocks*512 uint32. */
int atx_lds_probe(int mode, int blocks, int iters, unsigned* out, hipStream_t stream);

/* VALU issue rate of one instruction form: blocks x 512 threads, each lane
 * running 8 independent register chains of iters*8 instructions (64 per
 * lane per iteration) of form `mode`:
 *   0 v_add_u32;  1 v_add_u32_sdwa (sext WORD_1);  2 v_add_u32_sdwa (sext
 *   WORD_0);  3 v_bfe_i32;  4 v_pk_add_u16;  5 v_add3_u32;  6 v_perm_b32;
 *   7 v_dot2_i32_i16;  8 v_add_u32 and the mode-1 form alternating;
 *   9 v_xor_b32;  10 v_ashrrev_i32.
 * Instructions = blocks * 512 * iters * 64 (lane operations).  out:
 * blocks*512 uint32. */
int atx_valu_probe(int mode, int blocks, int iters, unsigned* out, hipStream_t stream);

/* The LUT GEMM's main loop without its global loads (lut_gemm_kernel's LDS
 * table layout, read addresses and pair adds; 128 accumulators per lane,
 * one 512-thread workgroup per CU).  mode = sum of: 1 the 16 table reads of
 * a sub-step, 2 the 128 adds, 4 the two table-build stores, 8 a barrier per
 * four sub-steps; modes 1, 2, 3, 4, 7, 11 and 15 are built.  Each iteration
 * is eight sub-steps of 128 lookups per lane: lookups = blocks * 512 * iters
 * * 8 * 128.  out: blocks*512 uint32. */
int atx_inner_probe(int mode, int blocks, int iters, unsigned* out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ATX_DIAG_H */
