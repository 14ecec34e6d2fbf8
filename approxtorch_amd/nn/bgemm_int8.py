"""int8 LUT BGEMM / LUT conv autograd Functions (STE, LRE, custom).

Forward: y[n,o,l] = sum_k lut[(x+128)*256 + (w+128)] on the gfx950 LUT GEMM.
Backward (all HIP):
  STE     the multiply is treated as exact on the quantized values;
  LRE     grad_x uses dx[idx(w)], grad_w uses dw[idx(x)] (256-entry tables);
  custom  grad_x uses dx_lut[idx(x)][idx(w)], grad_w dw_lut[idx(x)][idx(w)].
Mirrors approxtorch/nn/bgemm_int8.py (GEMM level 5-84, conv level 87-298).
Saved tensors are the uint8 index images (or the int8 image for the conv
level), never the fp32 operands.
"""
import torch
from torch.autograd import Function

from ..backend import ops

_TABLES = {}


def decode_table(device, signed=True):
    """[256] fp32 table idx -> quantized value (idx - 128 signed, idx unsigned)."""
    key = (str(device), signed)
    t = _TABLES.get(key)
    if t is None:
        t = torch.arange(256, device=device, dtype=torch.float32)
        if signed:
            t = t - 128
        _TABLES[key] = t
    return t


def _gemm_geom(N, K, L):
    # a [N, K, L] operand is the 1x1 im2col of an image [N, K, 1, L]
    return ops.L.geom(N, K, 1, L, 1, 1, 1, 1, 0, 0, 1, 1)


def _gemm_grads(go, xq, wq, tx, tw):
    """grad_x [N,K,L], grad_w [O,K] of sum_k f(x,w) with per-operand tables."""
    N, K, L = xq.shape
    O = wq.size(0)
    g = _gemm_geom(N, K, L)
    go = go.contiguous()
    col = torch.empty((N, K, L), dtype=torch.float32, device=go.device)
    ops.L.call("atx_conv_bwd_data_col", go.data_ptr(), wq.data_ptr(), tx.data_ptr(), N, O, K,
               L, col.data_ptr(), ops.L.stream_of(go))
    gw = ops.conv_backward_weight(go, xq.view(N, K, 1, L), tw, g, O, 128)
    return col, gw


class _bgemm_int8_base(Function):

    @staticmethod
    def forward(ctx, x, w, lut):
        y, xq, wq = ops.bgemm_fake_int8_claude_save(x, w, lut)
        ctx.save_for_backward(xq, wq)
        return y


class _bgemm_int8_ste(_bgemm_int8_base):
    """STE at GEMM level (nn/bgemm_int8.py:15-25): grad_x = W^T go, grad_w = go X^T
    on the quantized values (decoded from the saved index images)."""

    @staticmethod
    def backward(ctx, grad_output):
        xq, wq = ctx.saved_tensors
        dec = decode_table(xq.device)
        gx, gw = _gemm_grads(grad_output, xq, wq, dec, dec)
        return gx, gw, None


def bgemm_int8_ste(x, w, lut):
    return _bgemm_int8_ste.apply(x, w, lut)


class _bgemm_int8_lre(Function):
    """LRE at GEMM level (nn/bgemm_int8.py:29-52)."""

    @staticmethod
    def forward(ctx, x, w, lut, dx, dw):
        y, xq, wq = ops.bgemm_fake_int8_claude_save(x, w, lut)
        ctx.save_for_backward(xq, wq)
        ctx.dx, ctx.dw = dx, dw
        return y

    @staticmethod
    def backward(ctx, grad_outputs):
        xq, wq = ctx.saved_tensors
        gx, gw = _gemm_grads(grad_outputs, xq, wq, ctx.dx.contiguous(), ctx.dw.contiguous())
        return gx, gw, None, None, None


def bgemm_int8_lre(x, w, lut, dx, dw):
    return _bgemm_int8_lre.apply(x, w, lut, dx, dw)


class _bgemm_int8_custom(Function):
    """BGEMM with one custom derivative per quantized (x, w) pair
    (nn/bgemm_int8.py:55-84).  dx_lut / dw_lut are 256 x 256 row-major tables
    indexed [x + 128][w + 128]."""

    @staticmethod
    def forward(ctx, x, w, lut, dx_lut, dw_lut):
        y, xq, wq = ops.bgemm_fake_int8_claude_save(x, w, lut)
        ctx.save_for_backward(xq, wq, dx_lut, dw_lut)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        xq, wq, dx_lut, dw_lut = ctx.saved_tensors
        N, K, L = xq.shape
        grad_x, grad_w = ops.custom_grads(
            ops.pack_rows_u8(xq), wq, grad_output,
            dx_lut if ctx.needs_input_grad[0] else None,
            dw_lut if ctx.needs_input_grad[1] else None, N, K, L)
        return grad_x, grad_w, None, None, None


def bgemm_int8_custom(x, w, lut, dx_lut, dw_lut):
    return _bgemm_int8_custom.apply(x, w, lut, dx_lut, dw_lut)


# ------------------------------------------------------------- conv level
def _image(x):
    """The quantized image a conv Function reads: fp32 / int8 / uint8 as
    given; the integer values of an fp16 / bf16 fake-quantized x as int8
    (exact: |q| <= 128), the reference's `x.detach().to(torch.int8)`
    (nn/bgemm_int8.py:246)."""
    return x.detach().to(torch.int8) if x.dtype in ops.LOWP else x


def _conv_setup(x, w, geom):
    """Geometry and whether the conv is depthwise (groups == C == O, the only
    grouped form the reference supports: nn/Conv2d_int8.py:35-41)."""
    kernel_size, stride, padding, dilation, groups = geom
    g = ops.conv_geom(tuple(x.shape), kernel_size, stride, padding, dilation)
    if groups == 1:
        return g, False
    if groups == g.C and w.size(0) == g.C and w[0].numel() == g.KH * g.KW:
        return g, True
    raise NotImplementedError(
        "Conv2d_int8 supports groups=1 or depthwise (groups == in_channels == "
        f"out_channels), got groups={groups}, in={g.C}, out={w.size(0)}")


def _lut_conv(x, w, lut, g, depthwise):
    """LUT conv of the fp32 fake-quantized image x with fp32 quantized weights
    w [O, K]: (y [N, O, OH*OW], wq)."""
    if depthwise:
        wq, _, _ = ops._pack_w(w.reshape(g.C, -1).contiguous(), 128, want_wt=False)
        return ops.dwconv_forward(x, wq, lut, g, 128).view(g.N, g.C, -1), wq
    return ops.conv_forward(x, w, lut, g, 128, 128)


def _lut_conv_backward(go, xq8, wq, tx, tw, g, depthwise, **fused):
    """(grad_x, grad_w [O, K]) of the LUT conv under a per-operand table
    estimator; `fused` carries the go scale and fake-quant masks."""
    mx, sx_m = fused.get("mask"), fused.get("scale")
    mw, sw_m = fused.get("mask_w"), fused.get("scale_w")
    gsx, gsw = fused.get("go_sx"), fused.get("go_sw")
    if depthwise:
        gx = ops.dwconv_backward_data(go, wq, tx, g, mask=mx, scale=sx_m, go_sx=gsx, go_sw=gsw)
        gw = ops.dwconv_backward_weight(go, xq8, tw, g, 128, mask_w=mw, scale_w=sw_m,
                                        go_sx=gsx, go_sw=gsw)
        return gx, gw
    gx = ops.conv_backward_data(go, wq, tx, g, mask=mx, scale=sx_m, go_sx=gsx, go_sw=gsw)
    gw = ops.conv_backward_weight(go, xq8, tw, g, wq.size(0), 128, mask_w=mw, scale_w=sw_m,
                                  go_sx=gsx, go_sw=gsw)
    return gx, gw


class _conv2d_int8_ste(Function):
    """Conv-level STE (nn/bgemm_int8.py:229-297).  Forward: implicit-im2col LUT
    conv (or the depthwise LUT conv for groups == C) of the quantized image;
    saves the int8 image and uint8 weight indices.  Backward: fp32-MFMA
    backward-data (+ fold) and backward-weight on the decoded quantized values
    (zero padding decodes to 0)."""

    @staticmethod
    def forward(ctx, x, w, lut, geom):
        g, depthwise = _conv_setup(x, w, geom)
        y, wq = _lut_conv(_image(x), w, lut, g, depthwise)
        ctx.save_for_backward(x.detach().to(torch.int8), wq)
        ctx.g, ctx.depthwise = g, depthwise
        return y

    @staticmethod
    def backward(ctx, grad_outputs):
        xq8, wq = ctx.saved_tensors
        dec = decode_table(xq8.device)
        go = grad_outputs.contiguous()
        grad_x, grad_w = _lut_conv_backward(go, xq8, wq, dec, dec, ctx.g, ctx.depthwise)
        return grad_x, grad_w, None, None


def conv2d_int8_ste(x, w, lut, geom):
    return _conv2d_int8_ste.apply(x, w, lut, geom)


class _conv2d_int8_lre(Function):
    """Conv-level LRE (nn/bgemm_int8.py:126-214): grad_x = fold(W'^T go) with
    W' = dx[idx(w)], grad_w = go X'^T with X' = dw[idx(x)] and padded taps
    taking dw[128]."""

    @staticmethod
    def forward(ctx, x, w, lut, dx, dw, geom):
        g, depthwise = _conv_setup(x, w, geom)
        y, wq = _lut_conv(_image(x), w, lut, g, depthwise)
        ctx.save_for_backward(x.detach().to(torch.int8), wq)
        ctx.g, ctx.dx, ctx.dw, ctx.depthwise = g, dx, dw, depthwise
        return y

    @staticmethod
    def backward(ctx, grad_outputs):
        xq8, wq = ctx.saved_tensors
        go = grad_outputs.contiguous()
        grad_x, grad_w = _lut_conv_backward(go, xq8, wq, ctx.dx.contiguous(),
                                            ctx.dw.contiguous(), ctx.g, ctx.depthwise)
        return grad_x, grad_w, None, None, None, None


def conv2d_int8_lre(x, w, lut, dx, dw, geom):
    return _conv2d_int8_lre.apply(x, w, lut, dx, dw, geom)


class _conv2d_int8_fused(Function):
    """Conv2d_int8's forward and STE / LRE backward as one Function: the
    composition of nn/Conv2d_int8.py:192-212 (fake-quant of x and W, LUT conv,
    `addcmul(bias, y, scale_x * scale_w)`), the conv Functions above and the
    fake-quant Functions (nn/quantization.py:37-62,98-113), without the fp32
    fake-quantized tensors in between:
      forward:  x -> int8 image + mask, W -> uint8 GEMM operand + mask, LUT
                conv with the dequant epilogue bias + y * (scale_x * scale_w[o]);
      backward: go * (scale_x * scale_w[o]) applied in the MFMA operand loads,
                the x fake-quant STE fused into the fold (or the GEMM epilogue of
                a 1x1 conv), the W one into the split-K sum; grad_bias = sum go.
    tx / tw: the estimator's tables (STE: decode tables, LRE: dx / dw)."""

    @staticmethod
    def forward(ctx, x, weight, bias, scale_x, scale_w, lut, tx, tw, geom, qmin, qmax, qmax_w,
                x_upper=None, save_image=False):
        g, depthwise = _conv_setup(x, weight, geom)
        O = weight.size(0)
        # an fp16 / bf16 x: fake-quant in its dtype, the STE applied in it in
        # backward (the fused fp32 STE would round differently)
        lowp = x.dtype if x.dtype in ops.LOWP else None
        # a 1x1, stride-1, unpadded conv reads x itself as its operand: the
        # fake-quant writes the row-offset operand directly, no byte image
        pointwise = (lowp is None and not save_image and not depthwise and g.KH == 1 and
                     g.KW == 1 and g.SH == 1 and g.SW == 1 and g.PH == 0 and g.PW == 0)
        # weight_bits <= 4: indices w + 128 in [120, 136), matrix-core LUT GEMM
        wbase = 120 if qmax_w <= 7 else None
        # Without a flag from the statistic (eval mode, data parallel training)
        # the fake-quant reports whether every quantized x is >= 0 (LUT index
        # >= 128, the im2col's padding index included) for the LUT GEMM's
        # upper-half tables; only the gather kernel reads it.
        fq_flag = None
        if x_upper is None and not depthwise and wbase is None:
            x_upper = fq_flag = ops.upper_flag(x.device)
        if pointwise:
            mask_x, xt_rpad = ops.fakequant_rows(x, scale_x, qmin, qmax, 128, upper=fq_flag)
        else:
            _, mask_x, xq8 = ops.fakequant_per_tensor(x, scale_x, qmin, qmax, want_q=False,
                                                      q8_dtype=torch.int8, nonneg=fq_flag)
        mask_w, wq, wt, Opad = weight_pack(weight, scale_w, qmax_w, not depthwise)
        # addcmul(bias, y, s) promotes a low-precision bias to fp32 as well
        b = None if bias is None else bias.detach().float().contiguous()
        if pointwise:
            y, _ = ops.conv_forward_rows(xt_rpad, wq, lut, g, 128,
                                         out_kind=ops.L.ATX_OUT_DEQUANT, sx=scale_x,
                                         sw=scale_w, bias=b, packed_w=(wq, wt, Opad),
                                         wbase=wbase, x_upper=x_upper)
            saved_x, ctx.rpad = xt_rpad
        elif depthwise:
            y = ops.dwconv_forward(xq8, wq, lut, g, 128, out_kind=ops.L.ATX_OUT_DEQUANT,
                                   sx=scale_x, sw=scale_w, bias=b)
            saved_x, ctx.rpad = xq8, None
        elif save_image:
            # keep the int8 image (1 byte per input element); grad_w unfolds
            # it again in its loads
            y, _ = ops.conv_forward(
                xq8, wq, lut, g, 128, 128, out_kind=ops.L.ATX_OUT_DEQUANT, sx=scale_x,
                sw=scale_w, bias=b, packed_w=(wq, wt, Opad), wbase=wbase, x_upper=x_upper)
            saved_x, ctx.rpad = xq8, None
        else:
            # the row-offset operand is kept for the weight gradient: its
            # indices feed the backward GEMM with no im2col in the loop
            y, _, (xt, Rpad) = ops.conv_forward(
                xq8, wq, lut, g, 128, 128, out_kind=ops.L.ATX_OUT_DEQUANT, sx=scale_x,
                sw=scale_w, bias=b, packed_w=(wq, wt, Opad), return_operand=True,
                wbase=wbase, x_upper=x_upper)
            saved_x, ctx.rpad = xt, Rpad
        ctx.save_for_backward(saved_x, mask_x, wq, mask_w.view(O, -1), scale_x, scale_w,
                              tx.contiguous(), tw.contiguous())
        ctx.g, ctx.has_bias, ctx.wshape = g, bias is not None, weight.shape
        ctx.depthwise, ctx.lowp = depthwise, lowp
        return y.view(g.N, O, g.OH, g.OW)

    @staticmethod
    def backward(ctx, grad_output):
        saved_x, mask_x, wq, mask_w, sx, sw, tx, tw = ctx.saved_tensors
        g = ctx.g
        go = grad_output.contiguous()
        gx = gw = gb = None
        # fp32 x: the STE fused into the data gradient; fp16 / bf16 x: the
        # gradient wrt the quantized x in fp32, then the STE in x's dtype
        mx, msx = (None, None) if ctx.lowp else (mask_x, sx)
        if ctx.depthwise:
            if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
                gx, gw = _lut_conv_backward(go, saved_x, wq, tx, tw, g, True, mask=mx,
                                            scale=msx, mask_w=mask_w, scale_w=sw, go_sx=sx,
                                            go_sw=sw)
                gx = gx if ctx.needs_input_grad[0] else None
                gw = gw.view(ctx.wshape) if ctx.needs_input_grad[1] else None
        else:
            if ctx.needs_input_grad[0]:
                gx = ops.conv_backward_data(go, wq, tx, g, mask=mx, scale=msx, go_sx=sx,
                                            go_sw=sw)
            if ctx.needs_input_grad[1] and ctx.rpad is None:
                gw = ops.conv_backward_weight(go, saved_x, tw, g, wq.size(0), 128,
                                              mask_w=mask_w, scale_w=sw, go_sx=sx,
                                              go_sw=sw).view(ctx.wshape)
            elif ctx.needs_input_grad[1]:
                gw = ops.conv_backward_weight_rows(go, (saved_x, ctx.rpad), tw, g, wq.size(0),
                                                   mask_w=mask_w, scale_w=sw, go_sx=sx,
                                                   go_sw=sw).view(ctx.wshape)
        if gx is not None and ctx.lowp:
            gx = ops.fakequant_per_tensor_backward(gx.view(mask_x.shape), mask_x, sx,
                                                   dtype=ctx.lowp)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            gb = go.sum(dim=(0, 2, 3))
        return gx, gw, gb, None, None, None, None, None, None, None, None, None, None, None


def weight_pack(weight, scale_w, qmax_w, want_wt=True):
    """The fused layer's weight operand: per-channel fake-quant of W to
    indices w + 128 in [-qmax_w, qmax_w] + 128 (mask, wq [O, K], the transposed
    GEMM operand wt or None, Opad), no fp32 fake-quantized copy.  Per-channel
    scales promote an fp16 / bf16 weight's x / s to fp32
    (nn/quantization.py:100-105): the fp32 kernels run on its exact values."""
    _, mask_w, wq, wt, Opad = ops.fakequant_per_channel(weight.detach().float(), scale_w,
                                                        -qmax_w, qmax_w, offset=128,
                                                        want_wt=want_wt, want_q=False)
    return mask_w, wq, wt, Opad


def conv2d_int8_fused(x, weight, bias, scale_x, scale_w, lut, tx, tw, geom, qmin, qmax,
                      qmax_w, x_upper=None, save_image=False):
    """x_upper: optional device int32 flag, written for this same x, that is
    nonzero only when x >= 0 everywhere (Conv2d_int8's training-mode statistic,
    atx_absmax_ema_upper); the LUT GEMM then builds half-height tables.  The
    promise x >= 0 => every quantized x >= 0 holds because the fake-quant
    divides by max(scale_x, 1e-12) > 0 and qmax >= 0.  Without it, the
    fake-quant writes such a flag from the quantized values themselves.
    save_image: keep the int8 image for grad_w instead of the row-offset
    operand (less memory; grad_w unfolds the image in its loads)."""
    if qmax < 0 or qmin > qmax:
        raise RuntimeError(f"qmin/qmax must satisfy qmin <= qmax and qmax >= 0, got "
                           f"[{qmin}, {qmax}]")
    return _conv2d_int8_fused.apply(x, weight, bias, scale_x, scale_w, lut, tx, tw, geom,
                                    qmin, qmax, qmax_w, x_upper, save_image)


class _conv2d_int8_custom(Function):
    """Conv wrapper of the pair-wise custom-gradient kernels
    (nn/bgemm_int8.py:87-123).  The reference saves the unfolded uint8 index
    image; here the forward's row-offset operand (the implicit im2col's
    output, padded taps at index 128) is saved and read by the gradient
    kernels directly."""

    @staticmethod
    def forward(ctx, x, w, lut, dx_lut, dw_lut, geom, qmax_w=None):
        kernel_size, stride, padding, dilation, groups = geom
        if groups != 1:
            raise NotImplementedError("custom gradient currently supports only groups=1")
        g, _ = _conv_setup(x, w, geom)
        # w quantized to [-qmax_w, qmax_w] with qmax_w <= 7 (weight_bits <= 4): indices
        # w + 128 lie in [120, 136); the LUT GEMM and grad_x run on the matrix cores
        ctx.wbase = 120 if qmax_w is not None and qmax_w <= 7 else None
        y, wq, (xt, Rpad) = ops.conv_forward(_image(x), w, lut, g, 128, 128,
                                             return_operand=True, wbase=ctx.wbase)
        ctx.save_for_backward(xt, wq, dx_lut, dw_lut)
        ctx.g, ctx.rpad = g, Rpad
        return y

    @staticmethod
    def backward(ctx, grad_output):
        xt, wq, dx_lut, dw_lut = ctx.saved_tensors
        g = ctx.g
        grad_col, grad_w = ops.custom_grads(
            (xt, ctx.rpad), wq, grad_output, dx_lut if ctx.needs_input_grad[0] else None,
            dw_lut if ctx.needs_input_grad[1] else None, g.N, g.C * g.KH * g.KW, g.OH * g.OW,
            wbase=ctx.wbase)
        grad_x = ops.col2im(grad_col, g) if grad_col is not None else None
        return grad_x, grad_w, None, None, None, None, None


def conv2d_int8_custom(x, w, lut, dx_lut, dw_lut, geom, qmax_w=None):
    """qmax_w (optional): w holds values quantized to [-qmax_w, qmax_w]."""
    return _conv2d_int8_custom.apply(x, w, lut, dx_lut, dw_lut, geom, qmax_w)
