/*
 * atx.h — C ABI of the MI355X (gfx950) LUT approximate-multiplier library.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t,
 * launches HIP kernels on that stream, never allocates device memory itself
 * (workspaces are passed in by the caller) and never throws.  Return value:
 * ATX_OK (0) or a negative ATX_E* code; atx_last_error() returns a message for
 * the last failure on the calling thread.  Reference citations below are
 * relative to the ApproxTorch tree (approxtorch/backend/csrc = csrc/).
 *
 * Index conventions (shared with the reference, csrc/naive_cuda/README.md:17-35):
 *   LUT is a flat fp32 [65536] table, entry [xi * 256 + wi]; the activation
 *   operand selects the row.  int8 operands index as v + 128, uint8 as v.
 */
#ifndef ATX_H
#define ATX_H

#include <stdint.h>
#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ATX_OK = 0,
  ATX_EINVAL = -1,   /* bad argument (shape, size, null pointer) */
  ATX_ELAUNCH = -2,  /* a kernel launch or HIP runtime call failed */
  ATX_ERANGE = -3,   /* problem larger than the kernel's documented limits */
};

/* LUT image classes returned by atx_lut_prepare (flags on the device). */
enum {
  ATX_LUT_I16 = 0,   /* every entry is an integer in [-32767, 32767]   */
  ATX_LUT_U16 = 1,   /* every entry is an integer in [0, 65535]        */
  ATX_LUT_F32 = 2,   /* anything else: fp32 accumulation fallback      */
};

/* Element types of activations read by the *_dt entry points. */
enum {
  ATX_DT_F32 = 0,
  ATX_DT_F16 = 1,    /* IEEE binary16                 */
  ATX_DT_BF16 = 2,   /* bfloat16 (the high half of an fp32) */
};

/* Convolution geometry (NCHW input, OIHW weight). */
typedef struct atx_conv_geom {
  int N, C, H, W;          /* input image                       */
  int KH, KW;              /* kernel                            */
  int SH, SW, PH, PW, DH, DW;
  int OH, OW;              /* output spatial size               */
} atx_conv_geom;

/* ABI version, returned by atx_version().  2: atx_gemm_epilogue carries
 * its own size (first field) and the x_upper flag; atx_custom_grad_dx/dw
 * take the dy_scale and dx/dw table arguments below and atx_tap_sum its
 * workspace; atx_fakequant_fwd/rows and the row packers (atx_pack_x_f32/u8,
 * atx_pack_rows_strided) take a nullable upper-half flag.  Version 1
 * callers must be rebuilt against this header. */
#define ATX_ABI_VERSION 2

const char* atx_last_error(void);
int atx_version(void);

/* Measurement hook (no counterpart in the reference; bench.py's kernel
 * timer): while set on the calling thread, atx_lut_gemm,
 * atx_lut_gemm_noalloc and atx_lut_gemm_narrow record `before` on their
 * stream right before their main kernel (lut_gemm_kernel, lut_f32_kernel for
 * the fp32 class, onehot_gemm_kernel) and `after` right after it, not around
 * the split-K reduce or stream-K clear / finish launches, so that
 * hipEventElapsedTime gives that kernel's own duration.  Each call records
 * the pair again; set both to null to stop.  Both or neither. */
int atx_set_timing_events(hipEvent_t before, hipEvent_t after);

/* ---------------------------------------------------------------- LUT image
 * Re-encodes an fp32 LUT into the 16-bit transposed image used by the
 * LUT GEMM: out16t[wi * 256 + xi] = low 16 bits of lut[xi * 256 + wi]; also
 * writes the fp32 transposed copy outf32t (same layout) and flags[2]:
 * flags[0] = 1 if some entry is not an exact int16, flags[1] = 1 if some entry
 * is not an exact uint16.  flags must be zeroed by the caller beforehand.
 * Replaces prepare_lut_kernel (csrc/claude/bgemm_lut_kernels.cuh:116-142),
 * which the reference re-runs inside every forward call
 * (csrc/claude/bgemm_float_claude.cu:161-192). */
int atx_lut_prepare(const float* lut, uint16_t* out16t, float* outf32t,
                    int* flags, hipStream_t stream);

/* --------------------------------------------------------- operand packing
 * The LUT GEMM reads its activation operand as "row offsets": a
 * [Kpad][Rpad] uint16 array (R = N*L rows, Rpad = R rounded up to
 * ATX_ROW_TILE, Kpad = K rounded up to 4) whose entry for LUT index v is
 * atx_row_offset(v).  The k-rows come in quads rotated per row: slot s of a
 * quad holds, for row r, tap k = (s & ~3) | (((r >> 2) + s) & 3)
 * (atx_operand_tap).  Padding rows and taps k >= K hold offset 0.
 */
#define ATX_ROW_TILE 2048
#define ATX_COL_TILE 32

/* x fp32 [N,K,L] holding quantized integer values -> xq uint8 [N,K,L]
 * (LUT index clamp(rint(v) + offset, 0, 255), nullable) and the row-offset
 * operand xt [Kpad][Rpad].  upper (nullable, here and in the other row
 * packers): a device int the caller sets nonzero beforehand, cleared when an
 * index written for rows below N*L and taps below K is under 128; nonzero
 * afterwards, it is the promise atx_gemm_epilogue.x_upper takes for xt.
 * Replaces quantize_to_u8_kernel (csrc/claude/bgemm_lut_kernels.cuh:62-97)
 * for the x operand. */
int atx_pack_x_f32(const float* x, int N, int K, int L, int offset,
                   uint8_t* xq, uint16_t* xt, int Rpad, int* upper, hipStream_t stream);

/* x uint8 [N,K,L] (already LUT indices) -> row-offset operand xt. */
int atx_pack_x_u8(const uint8_t* xq, int N, int K, int L,
                  uint16_t* xt, int Rpad, int* upper, hipStream_t stream);

/* w fp32 [O,K] quantized values -> wq uint8 [O,K] (LUT index) and the
 * transposed, column-padded operand wt uint8 [K][Opad] (Opad = O rounded up
 * to ATX_COL_TILE; padding columns hold index 0); either output may be NULL,
 * not both (the depthwise conv needs wq alone).  Replaces the weight prepass
 * of csrc/claude/bgemm_float_claude.cu:108-130. */
int atx_pack_w_f32(const float* w, int O, int K, int offset,
                   uint8_t* wq, uint8_t* wt, int Opad, hipStream_t stream);

/* w uint8 [O,K] LUT indices -> wt uint8 [K][Opad]. */
int atx_pack_w_u8(const uint8_t* wq, int O, int K, uint8_t* wt, int Opad,
                  hipStream_t stream);

/* Operands of the plain (torch.mm-layout) LUT GEMM from strided 2-D inputs.
 * dtype 0: fp32 values, index clamp(rint(v) + offset, 0, 255); 1: uint8
 * indices.  Rows: X[r][k] at x + r*sr + k*sk -> xt [Kpad][Rpad] (as
 * atx_pack_x_u8, R rows) and the u8 image xq [R][K] (nullable).  Columns:
 * Y[c][k] at y + c*sc + k*sk -> wt [K][Opad] and yq [C][K] (nullable).
 * Replace the quantize and fused quantize-transpose prepasses of
 * csrc/claude/gemm.cu:57-100,128-166. */
int atx_pack_rows_strided(const void* x, int dtype, int R, int K, long long sr,
                          long long sk, int offset, uint8_t* xq, uint16_t* xt,
                          int Rpad, int* upper, hipStream_t stream);
int atx_pack_cols_strided(const void* y, int dtype, int C, int K, long long sc,
                          long long sk, int offset, uint8_t* yq, uint8_t* wt,
                          int Opad, hipStream_t stream);

/* Quantized image -> row-offset operand xt [Kpad][Rpad] (K = C*KH*KW) of the
 * implicit im2col, k order (c, kh, kw), r = n*OH*OW + oh*OW + ow.  dtype:
 * 0 = int8 values (index v+128), 1 = uint8 (index v), 2 = fp32 signed
 * quantized values (index clamp(rint(v),-128,127)+128), 3 = fp32 unsigned
 * quantized values (index clamp(rint(v),0,255)).  Out-of-image taps take LUT
 * index pad_index (128 = quantized zero for int8), or rint(pad_dev[0]) when
 * pad_dev is non-null (the device-resident uint8 zero point).
 * Replaces im2col_u8_kernel (csrc/claude/bgemm_lre_backward_claude.cu:215-269)
 * feeding the forward (nn/bgemm_int8.py:152-153). */
int atx_im2col_rows(const void* img, int dtype, atx_conv_geom g,
                    int pad_index, const float* pad_dev, uint16_t* xt, int Rpad,
                    hipStream_t stream);

/* The reference op im2col_u8 itself: image (int8 values, uint8 indices or
 * fp32 values; dtype 0 = int8, 1 = uint8, 2 = fp32) -> uint8 LUT indices
 * [N, C*KH*KW, OH*OW], padding -> index 128.
 * csrc/claude/bgemm_lre_backward_claude.cu:215-269 (kernel), 737-791 (host). */
int atx_im2col_u8(const void* img, int dtype, atx_conv_geom g, uint8_t* out,
                  hipStream_t stream);

/* ------------------------------------------------------------- LUT GEMM
 * y[n, o, l] = sum_k LUT[xi(n,k,l)][wi(o,k)], exact int32 accumulation,
 * for the operands produced by the pack / im2col entry points above.
 * lut16t / lutf32t come from atx_lut_prepare; lut_class selects the path
 * (ATX_LUT_I16 / ATX_LUT_U16: LDS-resident 16-bit tables, int32 sums;
 * ATX_LUT_F32: fp32 sums in ascending k, the reference's own order).
 * Epilogue (out_kind):
 *   ATX_OUT_F32     y fp32 [N,O,L] = (float) sum
 *   ATX_OUT_I32     y int32 [N,O,L] = sum  (integer classes only)
 *   ATX_OUT_DEQUANT y fp32 [N,O,L] = bias[o] + (float) sum * (sx[0]*sw[o])
 *                   (bias nullable)  — nn/Conv2d_int8.py:213-218 fused.
 * workspace: int32 scratch of atx_lut_gemm_workspace_bytes() bytes (split-K
 * partial sums, or the stream-K slots of tiles cut between workgroups:
 * 255 x 2048 x 32 int32); may be null when that function returns 0.  The
 * schedule (whole tiles, split-K, or whole-tile rounds then stream-K) is
 * chosen by a cost model; the environment variable ATX_LUT_SCHEDULE
 * (auto | split | stream_k) overrides it, read by both functions.
 * Replaces bgemm_lut_u8_kernel + reduce_splits_kernel + launch/dispatch
 * (csrc/claude/bgemm_lut_kernels.cuh:148-163,183-506). */
enum { ATX_OUT_F32 = 0, ATX_OUT_I32 = 1, ATX_OUT_DEQUANT = 2 };

typedef struct atx_gemm_epilogue {
  /* sizeof(atx_gemm_epilogue): set by atx_gemm_epilogue_make (or by hand).
   * Every entry point taking the struct rejects another value with
   * ATX_EINVAL before touching the device, so a caller built against an
   * older header (whose first field is out_kind, 0..2) fails cleanly. */
  int size;
  int out_kind;
  const float* scale_x;   /* [1]  (DEQUANT) */
  const float* scale_w;   /* [O]  (DEQUANT) */
  const float* bias;      /* [O] or null    */
  /* Device int or null, read by atx_lut_gemm / atx_lut_gemm_noalloc at
   * kernel start (atx_lut_gemm_narrow ignores it): nonzero promises that
   * every activation index of the rows below N*L is at least 128, as for the
   * int8 operand of an x >= 0 (atx_absmax_ema_upper writes such a flag;
   * atx_fakequant_fwd / atx_fakequant_rows and the row packers derive one
   * from the quantized indices themselves).
   * The kernel then builds only rows 128..255 of its tables, half the table
   * work, with the same exact sums; a broken promise gives wrong sums, never
   * an out-of-bounds access.  No counterpart in the reference. */
  const int* x_upper;
} atx_gemm_epilogue;

static inline atx_gemm_epilogue atx_gemm_epilogue_make(int out_kind, const float* scale_x,
                                                       const float* scale_w,
                                                       const float* bias,
                                                       const int* x_upper) {
  atx_gemm_epilogue ep;
  ep.size = (int)sizeof(atx_gemm_epilogue);
  ep.out_kind = out_kind;
  ep.scale_x = scale_x;
  ep.scale_w = scale_w;
  ep.bias = bias;
  ep.x_upper = x_upper;
  return ep;
}

long long atx_lut_gemm_workspace_bytes(int N, int K, int L, int O);

int atx_lut_gemm(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                 int N, int K, int L, int O,
                 const uint16_t* lut16t, const float* lutf32t, int lut_class,
                 atx_gemm_epilogue ep, void* y, void* workspace,
                 hipStream_t stream);

/* atx_lut_gemm for weights with at most 16 distinct indices: every wt entry
 * of the O channels lies in [wbase, wbase + 16) (weight_bits <= 4: wbase 0
 * for uint8 indices, 120 for int8 values v + 128); integer LUT classes only.
 * The sum is regrouped by weight index into a product with a 0/1 operand on
 * the int8 matrix cores, the 16-bit entries in two exact int8 planes: the
 * same exact int32 sums as atx_lut_gemm (entries outside the range give wrong
 * sums, never an out-of-bounds access).  Same operands, epilogues and output;
 * workspace of atx_lut_gemm_narrow_workspace_bytes() (split-K partials).
 * Replaces the reference's LUT GEMM (csrc/claude/bgemm_lut_kernels.cuh:
 * 183-387, host bgemm_float_claude.cu:80-240) for the weight_bits <= 4 layers
 * (nn/Conv2d_uint8.py:257-325, nn/Conv2d_int8.py:178-232). */
long long atx_lut_gemm_narrow_workspace_bytes(int N, int K, int L, int O);
int atx_lut_gemm_narrow(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                        int N, int K, int L, int O, const uint16_t* lut16t, int lut_class,
                        int wbase, atx_gemm_epilogue ep, void* y, void* workspace,
                        hipStream_t stream);

/* atx_lut_gemm_narrow (wbase 0: uint8 weight indices in [0, 16)) with the
 * uint8 layer's zero-point correction and dequant as its epilogue, the
 * in-place pass of atx_uint8_dequant folded into the GEMM's stores:
 *   y[n,o,l] = ((S - zero_w[o]*xsum[n,l] - zero_x*wsum[o] + K*zero_x*zero_w[o])
 *               * (scale_x * scale_w[o])) (+ bias[o], nullable)
 * for the exact sum S, each fp32 operation in atx_uint8_dequant's order, so
 * y is bit for bit the F32 GEMM followed by atx_uint8_dequant.  xsum
 * [N*L] = atx_tap_sum of the uint8 image, wsum[o] = sum_k q_w[o,k].  K > 0;
 * same workspace as atx_lut_gemm_narrow.  Replaces the LUT conv and the
 * correction / dequant tail of nn/Conv2d_uint8.py:257-325. */
int atx_lut_gemm_narrow_uint8(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                              int N, int K, int L, int O, const uint16_t* lut16t,
                              int lut_class, const float* scale_x, const float* scale_w,
                              const float* bias, const float* xsum, const float* wsum,
                              const float* zero_x, const float* zero_w, float* y,
                              void* workspace, hipStream_t stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory -- code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc.  atx_lut_gemm with the same arguments and results, minus
 * the workspace: split-K partial sums and stream-K slots live in a
 * library-owned static device array of ATX_NOALLOC_SCRATCH_BYTES (64 MiB),
 * one per GPU, held until the process ends.  The schedule is restricted to
 * those whose workspace fits it (stream-K slots always do; split counts
 * whose partials would not are skipped, which can change the speed but not
 * the exact int32 sums); when the int32-exactness bound forces a split that
 * does not fit (K > 32768 with R*O*4*ceil(K/32768) > 64 MiB) it returns
 * ATX_ERANGE without launching.  It allocates nothing and calls no
 * allocating routine.  The stream must belong to the current device.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (concurrent streams, threads) race and must be serialized by the caller. */
#define ATX_NOALLOC_SCRATCH_BYTES (64LL << 20)
int atx_lut_gemm_noalloc(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                         int N, int K, int L, int O,
                         const uint16_t* lut16t, const float* lutf32t, int lut_class,
                         atx_gemm_epilogue ep, void* y, hipStream_t stream);

/* ------------------------------------------------------------ fake-quant
 * Per-tensor fake-quant, fused: q = clamp(rint(x / max(s,1e-12) [+ z]),
 * qmin, qmax) (NaN passes through), mask = qmin <= v <= qmax on the
 * pre-round v.  zero may be null (symmetric).  q and mask may each be null.
 * q8 (nullable): the same value as a signed/unsigned byte image.
 * nonneg (nullable): a device int the caller sets nonzero beforehand; the
 * kernel sets it to 0 when some quantized value is negative (NaN counts as
 * 0).  For the int8 operand (LUT index q + 128) a nonzero flag afterwards is
 * the promise atx_gemm_epilogue.x_upper takes; it is a property of the
 * quantized values themselves, whatever the scale.
 * csrc/claude/quantization.cu:54-75,77-110,148-183 (kernels), 187-311 (host). */
int atx_fakequant_fwd(const float* x, long long n, const float* scale,
                      const float* zero, int qmin, int qmax, float* q,
                      uint8_t* mask, void* q8, int* nonneg, hipStream_t stream);

/* The input fake-quant of a 1x1, stride-1, unpadded, ungrouped conv fused
 * with its operand packing: x fp32 [N,K,L] -> mask uint8 [N,K,L] (as
 * atx_fakequant_fwd) and the row-offset operand xt [Kpad][Rpad] whose LUT
 * index for x[n][k][l] is (q + offset) & 255, q the quantized value as an
 * integer (offset 128: the int8 byte image read with index v+128; 0: the
 * uint8 one).  Bit-identical to atx_fakequant_fwd's q8 followed by
 * atx_im2col_rows of that 1x1 geometry, without the byte image.  Replaces
 * the fake-quant of x (nn/quantization.py:37-62) and the im2col prepass
 * (csrc/claude/bgemm_lre_backward_claude.cu:215-269) of a 1x1 conv in
 * nn/Conv2d_int8.py:192-212.  upper (nullable): a device int the caller sets
 * nonzero beforehand; cleared when some index written for rows below N*L and
 * taps below K is under 128, so that afterwards it is the promise
 * atx_gemm_epilogue.x_upper takes for this operand. */
int atx_fakequant_rows(const float* x, int N, int K, int L, const float* scale,
                       const float* zero, int qmin, int qmax, int offset,
                       uint8_t* mask, uint16_t* xt, int Rpad, int* upper,
                       hipStream_t stream);

/* Per-tensor fake-quant of an fp16 / bf16 x (dtype ATX_DT_F16 or
 * ATX_DT_BF16), the reference's unfused statements for a non-fp32 input
 * (nn/quantization.py:44-52,72-80) as torch evaluates them in x's dtype D:
 * s = max(scale, 1e-12) cast to D; v = x / s rounded to D (+ zero cast to D,
 * rounded to D); mask = qmin <= v <= qmax; q = clamp(round(v), qmin, qmax)
 * in D (nullable).  mask, q8 and nonneg as atx_fakequant_fwd. */
int atx_fakequant_fwd_dt(const void* x, int dtype, long long n, const float* scale,
                         const float* zero, int qmin, int qmax, void* q, uint8_t* mask,
                         void* q8, int* nonneg, hipStream_t stream);

/* Its backward, gx = go * mask / s in D (nn/quantization.py:58-62,86-91):
 * go of go_dtype ATX_DT_F32 (rounded to D first, as autograd casts a
 * gradient to its input's dtype) or D; the product with the mask exact (a
 * 0 * inf is NaN), the quotient by s cast to D rounded to D. */
int atx_fakequant_bwd_dt(const void* go, int go_dtype, const uint8_t* mask, long long n,
                         const float* scale, int dtype, void* gx, hipStream_t stream);

/* gx = (mask ? go : 0) / max(scale, 1e-12); scale has 1 (per-tensor) or
 * C (per-channel, channel = (i / inner) % C) elements.
 * csrc/claude/quantization.cu:112-143; nn/quantization.py:110-113. */
int atx_fakequant_bwd(const float* go, const uint8_t* mask, long long n,
                      const float* scale, int C, long long inner, float* gx,
                      hipStream_t stream);

/* Per-channel fake-quant of a weight [O, inner]: q, mask, and the LUT index
 * image wq = q + offset (nullable), the transposed operand wt [inner][Opad]
 * (nullable, 4-byte aligned).  nn/quantization.py:98-133. */
int atx_fakequant_channel_fwd(const float* w, int O, long long inner,
                              const float* scale, const float* zero,
                              int qmin, int qmax, int offset, float* q,
                              uint8_t* mask, uint8_t* wq, uint8_t* wt,
                              int Opad, hipStream_t stream);

/* col2im (F.fold): img[n,c,h,w] = sum of col[n,(c,kh,kw),(oh,ow)] over the
 * taps that read (h,w).  If mask is non-null the per-tensor fake-quant
 * backward is fused: img = mask ? img / max(scale[0],1e-12) : 0.
 * nn/bgemm_int8.py:116-118 (F.fold) + csrc/claude/quantization.cu:112-143. */
int atx_col2im(const float* col, atx_conv_geom g, const uint8_t* mask,
               const float* scale, float* img, hipStream_t stream);

/* atx_col2im plus a per-position term: pos [N, OH*OW] fp32 (nullable) adds,
 * summed separately in the same tap order, sum of pos[n,(oh,ow)] over the
 * taps that read (h,w) -- the backward of a term broadcast to every tap of an
 * output position (tap_sum's backward) -- before the fused STE.  One pass for
 * nn/Conv2d_uint8.py:308-325's zero-point term z_w * sum_k q_x (its image
 * gradient) with F.fold of the main term and the STE of
 * csrc/claude/quantization.cu:223-258. */
int atx_col2im_pos(const float* col, atx_conv_geom g, const float* pos,
                   const uint8_t* mask, const float* scale, float* img,
                   hipStream_t stream);

/* Column sums of the unfolded image (dtype 1 = uint8 values, 2 = fp32
 * holding quantized integers), out[n,l] = sum over the K taps (out-of-image
 * taps count as pad_dev[0], 0 if null), exact; workspace:
 * atx_tap_sum_workspace_bytes(g) (per-64-channel sums).  And its backward
 * img[n,c,h,w] = sum of go[n,l] over the taps reading (h,w).  The uint8
 * zero-point correction term sum_k q_x of nn/Conv2d_uint8.py:308-315. */
/* Zero-point correction and dequant of a uint8 conv's raw LUT sums y
 * [N,O,L], in place:
 *   y = ((y - zero_w[o]*xsum[n,l] - zero_x*wsum[o] + K*zero_x*zero_w[o])
 *        * (scale_x * scale_w[o])) (+ bias[o], nullable),
 * each fp32 operation in that order; xsum = atx_tap_sum of the uint8 image,
 * wsum[o] = sum_k q_w[o,k].  Replaces the elementwise tail of
 * nn/Conv2d_uint8.py:308-325. */
int atx_uint8_dequant(float* y, int N, int O, int L, const float* xsum, const float* wsum,
                      const float* zero_x, const float* zero_w, const float* scale_x,
                      const float* scale_w, const float* bias, int K, hipStream_t stream);

long long atx_tap_sum_workspace_bytes(atx_conv_geom g);
int atx_tap_sum(const void* img, int dtype, atx_conv_geom g, const float* pad_dev,
                float* out, float* workspace, hipStream_t stream);
int atx_tap_sum_bwd(const float* go, atx_conv_geom g, float* img,
                    hipStream_t stream);

/* The backward of the uint8 zero-point term z_w[o] * sum_k q_x at each
 * output position: pos[n,l] = sum_o -(scale_x * scale_w[o]) * zero_w[o] *
 * go[n,o,l] (go [N,O,L]), fp32 products in that order, summed in a fixed
 * order (deterministic).  Its image gradient is atx_tap_sum_bwd /
 * atx_col2im_pos of pos.  Replaces the [1 x O] by [O x L] product of the
 * reference's autograd through nn/Conv2d_uint8.py:308-315. */
int atx_zero_point_pos(const float* go, int N, int O, int L, const float* scale_x,
                       const float* scale_w, const float* zero_w, float* pos,
                       hipStream_t stream);

/* Both reductions of go [N,O,L] that the uint8 layer's backward needs, in
 * one pass over go: pos as atx_zero_point_pos (nullable: then only the
 * sums), and gsum[o] = sum_{n,l} go[n,o,l] (O <= 8192), the gradient that
 * reaches the -z_x * sum_k q_w[o,k] term and the bias.  Each block of
 * positions is summed in a fixed lane order, each persistent workgroup's
 * blocks in order, and the workgroups' totals in a fixed order
 * (deterministic).  gsum == NULL: atx_zero_point_pos.  workspace:
 * atx_zero_point_terms_workspace_bytes(N, O, L) bytes.  Replaces go.sum over
 * (n, l) in the reference's autograd through nn/Conv2d_uint8.py:312-315
 * (the zero_x * wsum term) and :320-321 (the bias). */
long long atx_zero_point_terms_workspace_bytes(int N, int O, int L);
int atx_zero_point_terms(const float* go, int N, int O, int L, const float* scale_x,
                         const float* scale_w, const float* zero_w, float* pos, float* gsum,
                         float* workspace, hipStream_t stream);

/* --------------------------------------------------------------- EMA stats
 * absmax EMA (nn/Conv2d_int8.py:137-146):
 *   stat = max|x|; scale <- m*(stat/denom) + (1-m)*scale, in fp32 with
 *   torch's operation order.  ws: atx_reduce_workspace_bytes() of scratch.
 *   The statistic is written to stat_out, so a caller can all-reduce it
 *   between atx_absmax and atx_ema_absmax_apply (data parallel). */
long long atx_reduce_workspace_bytes(void);
int atx_absmax(const float* x, long long n, unsigned int* ws, float* stat_out,
               hipStream_t stream);
int atx_minmax(const float* x, long long n, unsigned int* ws, float* mn_out,
               float* mx_out, hipStream_t stream);
/* scale[0] <- m32 * (stat[0] / denom) + om32 * scale[0] */
int atx_ema_absmax_apply(const float* stat, float denom, float m32, float om32,
                         float* scale, hipStream_t stream);
/* atx_absmax then atx_ema_absmax_apply in one less launch (the EMA is applied
 * by the reduction's final block); same results.  For callers with no
 * all-reduce of the statistic in between (single process). */
int atx_absmax_ema(const float* x, long long n, unsigned int* ws, float* stat_out,
                   float denom, float m32, float om32, float* scale, hipStream_t stream);
/* atx_absmax_ema that also writes *upper = 1 when min(x) >= 0 (no NaN), else
 * 0: then the int8 fake-quant of x has every LUT index at or above 128, the
 * promise of atx_gemm_epilogue.x_upper, because the fake-quant divides by
 * max(scale, 1e-12) > 0 whatever the scale holds and its qmax is >= 0 (a
 * qmax < 0 would map x >= 0 below index 128: the caller must not use the
 * flag then).  Same stat_out
 * and scale update as atx_absmax_ema, bit for bit (max |x| is taken as
 * max(-min x, max x)).  No counterpart in the reference; used by the int8
 * layer's training-mode forward (nn/Conv2d_int8.py:137-146). */
int atx_absmax_ema_upper(const float* x, long long n, unsigned int* ws, float* stat_out,
                         float denom, float m32, float om32, float* scale, int* upper,
                         hipStream_t stream);
/* The absmax statistic and EMA of an activation x of any ATX_DT_* dtype
 * (nn/Conv2d_int8.py:137-146 evaluated by torch in x's dtype D): stat =
 * max|x| (exact), cur = stat / denom and m * cur rounded to D (abs_max is a
 * D scalar), (1 - m) * scale and the sum in fp32.  ATX_DT_F32 gives the
 * fp32 entry points' results.  No counterpart in the reference's kernels:
 * its layer runs these statements in torch for a non-fp32 x. */
int atx_absmax_dt(const void* x, int dtype, long long n, unsigned int* ws, float* stat_out,
                  hipStream_t stream);
int atx_ema_absmax_apply_dt(const float* stat, int dtype, float denom, float m32, float om32,
                            float* scale, hipStream_t stream);
int atx_absmax_ema_upper_dt(const void* x, int dtype, long long n, unsigned int* ws,
                            float* stat_out, float denom, float m32, float om32, float* scale,
                            int* upper, hipStream_t stream);
/* atx_minmax then atx_ema_minmax_apply, fused the same way. */
int atx_minmax_ema(const float* x, long long n, unsigned int* ws, float* mn_out,
                   float* mx_out, float m32, float om32, int qmax, float* x_min,
                   float* x_max, float* scale, float* zero, hipStream_t stream);
/* uint8 activation qparams (nn/Conv2d_uint8.py:11-23,225-240): EMA of
 * min/max then scale = max((mx'-mn')/qmax, 1e-12), zero = clamp(rint(-mn'/scale)). */
int atx_ema_minmax_apply(const float* mn, const float* mx, float m32, float om32,
                         int qmax, float* x_min, float* x_max, float* scale,
                         float* zero, hipStream_t stream);
/* Per-channel weight absmax EMA (nn/Conv2d_int8.py:148-158); a zero channel
 * keeps its old scale.  mode 1 = reset (nn/Conv2d_int8.py:160-167). */
int atx_weight_scale_ema(const float* w, int O, long long inner, float qmax_w,
                         float m32, float om32, int reset, float* scale_w,
                         hipStream_t stream);
/* atx_weight_scale_ema over a weight of any ATX_DT_* dtype: for fp16 / bf16
 * absmax / qmax_w is rounded to that dtype, as torch computes it for such a
 * weight (nn/Conv2d_int8.py:155,166); the EMA itself stays fp32. */
int atx_weight_scale_ema_dt(const void* w, int dtype, int O, long long inner, float qmax_w,
                            float m32, float om32, int reset, float* scale_w,
                            hipStream_t stream);
/* Per-channel weight min/max EMA + uint8 qparams (nn/Conv2d_uint8.py:242-255). */
int atx_weight_minmax_ema(const float* w, int O, long long inner, float m32,
                          float om32, int qmax, float* w_min, float* w_max,
                          float* scale_w, float* zero_w, hipStream_t stream);

/* ------------------------------------------------------------ LUT maps
 * out[i] = lut256[idx(in[i])], in dtype 0 int8 (v+128), 1 uint8 (v), 2 fp32
 * (clamp(rint(v),-128,127)+128).  csrc/claude/bgemm_lre_backward_claude.cu:95-127. */
int atx_lut_map(const void* in, int dtype, long long n, const float* lut256,
                float* out, hipStream_t stream);
/* image [N,C,H,W] -> [N,C,H+2PH,W+2PW], border = lut256[128].
 * csrc/claude/bgemm_lre_backward_claude.cu:276-307. */
int atx_lut_map_pad(const void* in, int dtype, int N, int C, int H, int W,
                    int PH, int PW, const float* lut256, float* out,
                    hipStream_t stream);

/* ------------------------------------------- STE / LRE backward (fp32 MFMA)
 * Backward of the LUT GEMM under an estimator that treats each product as
 * Tx[wi] * (something in go) and Tw[xi] * (...):
 *   col[n,k,l] = sum_o go[n,o,l] * tx[wq[o,k]]       (then atx_col2im)
 *   gw[o,k]    = sum_{n,l} go[n,o,l] * tw[xi(n,k,l)]
 * STE: tx/tw decode indices to quantized values; LRE: the dx / dw slope
 * tables.  xi is read from the saved image (dtype as atx_im2col_rows,
 * out-of-image taps -> tw[pad_index]).  go_sx/go_sw (nullable, together)
 * scale go by the fp32 product sx[0] * sw[o] first: the backward of the
 * layer's dequant y * (scale_x * scale_w).  mask_w/scale_w (nullable) fuse
 * the per-channel weight fake-quant backward.  Replace the cuBLAS / cuDNN
 * calls of csrc/claude/bgemm_lre_backward_claude.cu:443-524 and
 * nn/bgemm_int8.py:184-207,277-290. */
int atx_conv_bwd_data_col(const float* go, const uint8_t* wq, const float* tx,
                          int N, int O, int K, int L, float* col,
                          hipStream_t stream);
/* Image gradient of the conv: col as above (with the go scale), folded into
 * gx [N,C,H,W] with the per-tensor fake-quant STE fused when mask != NULL:
 * gx = (mask ? g : 0) / max(scale[0], 1e-12).  A 1x1 stride-1 unpadded conv
 * writes gx straight from the GEMM, and so does a stride-1 conv with
 * O % 32 == 0 whose C x N*H*W output fills >= 512 tiles (implicit GEMM over
 * (tap, o)); otherwise the workspace holds col.  When the output tiles
 * cannot fill the GPU the contraction over O is split into partial slices
 * (in the workspace) summed in a fixed order.  The workspace also holds the
 * tx[wq] values as bf16 parts for the matrix cores (the products are the
 * fp32 products to within 2^-20 relative; exact when tx holds bf16 values,
 * as the STE's integers do).  Size: atx_conv_bwd_data_workspace_bytes(g, O),
 * nonzero whenever O, K and L are.  Replaces the same calls
 * plus the fold and the fake-quant backward (nn/bgemm_int8.py:116-118,
 * csrc/claude/quantization.cu:223-258). */
long long atx_conv_bwd_data_workspace_bytes(atx_conv_geom g, int O);
int atx_conv_bwd_data(const float* go, const uint8_t* wq, const float* tx,
                      atx_conv_geom g, int O, const float* go_sx,
                      const float* go_sw, const uint8_t* mask,
                      const float* scale, float* gx, float* workspace,
                      hipStream_t stream);
long long atx_conv_bwd_weight_workspace_bytes(int O, int K, long long P);
/* atx_conv_bwd_weight with xi read from the forward's row-offset operand
 * xt [Kpad][Rpad] (as atx_im2col_rows / atx_pack_x_* wrote it; index =
 * entry >> 8, padding taps already hold the pad index): no implicit im2col
 * in the loop.  Rows r = n*L + l, P = N*L; same workspace as
 * atx_conv_bwd_weight. */
int atx_conv_bwd_weight_rows(const float* go, const uint16_t* xt, int Rpad,
                             int N, int K, int L, int O, const float* tw,
                             const float* go_sx, const float* go_sw,
                             const uint8_t* mask_w, const float* scale_w,
                             float* gw, float* workspace, hipStream_t stream);
int atx_conv_bwd_weight(const float* go, const void* img, int dtype,
                        atx_conv_geom g, int O, int pad_index,
                        const float* pad_dev, const float* tw,
                        const float* go_sx, const float* go_sw,
                        const uint8_t* mask_w, const float* scale_w, float* gw,
                        float* workspace, hipStream_t stream);

/* ----------------------------------------------- LUT files and gradient tables
 * Host: parses a text table (numbers separated by whitespace or commas, '#'
 * comments; integral != 0 rejects non-integers) into out[capacity]; *count
 * = values read.  Replaces the numpy.loadtxt calls of load_lut.py:5-55.
 * Device: LRE slope tables (grad_lut.py:14-37; offset 128 = int8 operands,
 * 0 = uint8) and DATE tables (grad_lut.py:39-142; half_ws in [0, 127],
 * grad_a/grad_b [65536] indexed like the LUT) of an fp32 LUT [65536]. */
int atx_parse_text_table(const char* path, int integral, float* out,
                         long long capacity, long long* count);
int atx_lre_tables(const float* lut, int offset, float* grad_a, float* grad_b,
                   hipStream_t stream);
int atx_date_tables(const float* lut, int half_ws, float* grad_a, float* grad_b,
                    hipStream_t stream);

/* ------------------------------------------------- depthwise LUT conv
 * groups == C == O: y[n,c,oh,ow] = sum_{i,j} LUT[xi(n,c,tap)][wq[c][i*KW+j]]
 * (taps in ascending (i, j); out-of-image taps -> index pad_index), exact
 * int32 for the integer LUT classes, fp32 in tap order for ATX_LUT_F32.
 * img dtype as atx_im2col_rows; wq [C][KH*KW] LUT indices; y [N,C,OH,OW]
 * with the atx_lut_gemm epilogues (sw / bias indexed by channel).  At most
 * 64 taps.  Replaces dwconv_fake_int8_claude
 * (csrc/claude/dwconv_claude.cu:1-285). */
int atx_dwconv_fwd(const void* img, int dtype, atx_conv_geom g, int pad_index,
                   const uint8_t* wq, const uint16_t* lut16t, const float* lutf32t,
                   int lut_class, atx_gemm_epilogue ep, void* y, hipStream_t stream);
/* STE / LRE backward of the depthwise conv (the grouped
 * convolution_backward of nn/bgemm_int8.py:162-212,259-295):
 *   gx[n,c,h,w] = sum over taps/outputs reading (h,w) of go' * tx[wq[c][t]]
 *   gw[c,t]     = sum_{n,oh,ow} go' * tw[xi(n,c,tap t)]
 * go' = go * fp32(sx[0] * sw[c]) when go_sx/go_sw are given; mask/scale and
 * mask_w/scale_w fuse the fake-quant STE as in atx_conv_bwd_data /
 * atx_conv_bwd_weight. */
int atx_dwconv_bwd_data(const float* go, const uint8_t* wq, const float* tx,
                        atx_conv_geom g, const float* go_sx, const float* go_sw,
                        const uint8_t* mask, const float* scale, float* gx,
                        hipStream_t stream);
long long atx_dwconv_bwd_weight_workspace_bytes(atx_conv_geom g);
int atx_dwconv_bwd_weight(const float* go, const void* img, int dtype,
                          atx_conv_geom g, int pad_index, const float* pad_dev,
                          const float* tw, const float* go_sx, const float* go_sw,
                          const uint8_t* mask_w, const float* scale_w, float* gw,
                          float* workspace, hipStream_t stream);

/* ------------------------------------------------------- custom gradients
 * Pair-table ("custom" estimator) gradients of the LUT GEMM:
 *   grad_x[n,k,l] = sum_o dy[n,o,l] * T[xi(n,k,l)][wi(o,k)]
 *   grad_w[o,k]   = sum_{n,l} dy[n,o,l] * T[xi(n,k,l)][wi(o,k)]
 * T a 256x256 fp32 table (the dx / dw table), passed transposed:
 * tabT[w * 256 + v] = T[v][w] (atx_lut_prepare's outf32t of T).  The
 * operands are the LUT GEMM's: xt [Kpad][Rpad] row offsets (as atx_pack_x_* /
 * atx_im2col_rows wrote them; rows r = n*L + l) and wt [K][Opad] indices.
 * dy [N,O,L] fp32; grad_x [N,K,L] fp32 (fold it with atx_col2im for a conv);
 * grad_w [O,K] fp32, with the per-channel weight fake-quant STE fused when
 * mask_w / scale_w are given (as atx_conv_bwd_weight).  dy_scale [O]
 * (nullable): the gradients of dy[n,o,l] * dy_scale[o] (each product rounded
 * once, as the caller's own multiply would), so a layer's per-channel output
 * scale needs no scaled copy of dy.  Table entries must
 * be finite.  Workspace of grad_w: atx_custom_grad_dw_workspace_bytes()
 * (one partial slice per 2048-row tile, summed in a fixed order).
 * Replace bgemm_custom_grad_{uint8,int8}_{dx,dw}
 * (csrc/cuda/bgemm_custom_grad_optimize.cu:30-116,136-205 uint8,
 * 315-404,419-490 int8; hosts 212-301,497-585). */
int atx_custom_grad_dx(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                       const float* dy, const float* tabT, int N, int K, int L, int O,
                       float* grad_x, hipStream_t stream);
long long atx_custom_grad_dw_workspace_bytes(int N, int K, int L, int O);
int atx_custom_grad_dw(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                       const float* dy, const float* dy_scale, const float* tabT, int N,
                       int K, int L, int O, const uint8_t* mask_w, const float* scale_w,
                       float* grad_w, float* workspace, hipStream_t stream);
/* atx_custom_grad_dw with the uint8 layer's weight zero-point term applied
 * before the STE: grad_w[o,k] = sum - (go_sum[o] * (scale_x * scale_w[o])) *
 * zero_x, each operation rounded on its own as the reference's elementwise
 * tensor ops round it, then the STE of mask_w / scale_w when mask_w is given.
 * go_sum[o] = sum_{n,l} go[n,o,l] (atx_zero_point_terms).  Replaces the
 * weight side of nn/Conv2d_uint8.py:308-325 after the custom gradient. */
int atx_custom_grad_dw_uint8(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                             const float* dy, const float* dy_scale, const float* tabT, int N,
                             int K, int L, int O, const uint8_t* mask_w, const float* scale_w,
                             const float* go_sum, const float* scale_x, const float* zero_x,
                             float* grad_w, float* workspace, hipStream_t stream);

/* atx_custom_grad_dx for weights with at most 16 distinct indices: every
 * wt entry of the O channels lies in [wbase, wbase + 16) (weight_bits <= 4:
 * wbase 0 for uint8 indices, 120 for int8 values v + 128).  The sum is
 * regrouped by weight index and runs on the bf16 matrix cores with dy split
 * exactly into three bf16 parts (fp32 sums, same error bound as
 * atx_custom_grad_dx; entries outside the range give wrong sums, never an
 * out-of-bounds access).  Same operands and output (dy_scale as in
 * atx_custom_grad_dw); Opad a multiple of 32.
 * Replaces bgemm_custom_grad_{uint8,int8}_dx for the weight_bits <= 4 layers
 * (csrc/cuda/bgemm_custom_grad_optimize.cu:30-116, 315-404; called from
 * nn/bgemm_uint8.py:89-114). */
int atx_custom_grad_dx_narrow(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                              const float* dy, const float* dy_scale, const float* tabT,
                              int wbase, int N, int K, int L, int O, float* grad_x,
                              hipStream_t stream);

/* atx_custom_grad_dx_narrow for a 1x1, stride-1, unpadded conv, whose
 * column gradient [N][K][L] is the image gradient [N][C][H*W]: the epilogue
 * also adds pos[n][l] (nullable) and applies the fake-quant STE (mask
 * [N][C][H][W] nullable, scale [1] with it), the operations and order of
 * atx_col2im_pos for that geometry, so the result equals
 * atx_custom_grad_dx_narrow followed by atx_col2im_pos bit for bit, without
 * the column buffer or the fold pass.  Replaces the same reference calls
 * for the uint8 layer's 1x1 convs (nn/bgemm_uint8.py:89-114 with the fold and
 * fake-quant backward of nn/Conv2d_uint8.py:308-325). */
int atx_custom_grad_dx_narrow_img(const uint16_t* xt, int Rpad, const uint8_t* wt, int Opad,
                                  const float* dy, const float* dy_scale, const float* tabT,
                                  int wbase, int N, int K, int L, int O, const float* pos,
                                  const uint8_t* mask, const float* scale, float* grad_img,
                                  hipStream_t stream);

#ifdef __cplusplus
}
#endif

/* Row-offset encoding of LUT index v used by the LUT GEMM's LDS tables
 * (256-byte lines; bits 4-5 carry the chunk swizzle (v >> 1) & 3). */
static inline unsigned atx_row_offset(unsigned v) {
  return v * 256u + (((v >> 1) & 3u) << 4);
}

/* Tap held by slot s of the row-offset operand for row r. */
static inline int atx_operand_tap(int s, int r) {
  return (s & ~3) | (((r >> 2) + s) & 3);
}

#endif /* ATX_H */
