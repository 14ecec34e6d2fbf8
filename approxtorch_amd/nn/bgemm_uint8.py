"""uint8 x uint8 LUT BGEMM autograd Functions (asymmetric quantization).

  y[n, o, l] = sum_k lut[x[n,k,l] * 256 + w[o,k]]   (raw values as indices)

The output is the raw LUT sum; the zero-point correction is the caller's
(Conv2d_uint8) job, written as differentiable ops so autograd adds the -z
terms.  Mirrors approxtorch/nn/bgemm_uint8.py:27-127 (GEMM level) and adds
conv-level Functions that run the implicit-im2col LUT conv on the quantized
image, with out-of-image taps taking the device-resident zero point (the
reference pads with z_x and unfolds in fp32, nn/Conv2d_uint8.py:283-294).
"""
import torch
from torch.autograd import Function

from ..backend import ops
from .bgemm_int8 import _gemm_grads, decode_table

__all__ = ["bgemm_uint8", "bgemm_uint8_ste", "bgemm_uint8_lre", "bgemm_uint8_custom",
           "conv2d_uint8_ste", "conv2d_uint8_lre", "conv2d_uint8_custom", "tap_sum",
           "conv2d_uint8_fused"]


class _bgemm_uint8_base(Function):

    @staticmethod
    def forward(ctx, x, w, lut):
        y, xq, wq = ops.bgemm_fake_uint8_claude_save(x, w, lut)
        ctx.save_for_backward(xq, wq)
        return y


class _bgemm_uint8_ste(_bgemm_uint8_base):
    """STE: d/dq_x = q_w, d/dq_w = q_x on the raw uint8 values
    (nn/bgemm_uint8.py:35-46)."""

    @staticmethod
    def backward(ctx, grad_output):
        xq, wq = ctx.saved_tensors
        ident = decode_table(xq.device, signed=False)
        gx, gw = _gemm_grads(grad_output, xq, wq, ident, ident)
        return gx, gw, None


def bgemm_uint8_ste(x, w, lut):
    return _bgemm_uint8_ste.apply(x, w, lut)


class _bgemm_uint8_lre(Function):
    """LRE with 256-entry tables indexed by the raw uint8 operand value
    (nn/bgemm_uint8.py:53-86)."""

    @staticmethod
    def forward(ctx, x, w, lut, dx, dw):
        y, xq, wq = ops.bgemm_fake_uint8_claude_save(x, w, lut)
        ctx.save_for_backward(xq, wq)
        ctx.dx, ctx.dw = dx, dw
        return y

    @staticmethod
    def backward(ctx, grad_output):
        xq, wq = ctx.saved_tensors
        gx, gw = _gemm_grads(grad_output, xq, wq, ctx.dx.contiguous(), ctx.dw.contiguous())
        return gx, gw, None, None, None


def bgemm_uint8_lre(x, w, lut, dx, dw):
    return _bgemm_uint8_lre.apply(x, w, lut, dx, dw)


class _bgemm_uint8_custom(Function):
    """Pair-wise custom derivatives dx_lut[x][w], dw_lut[x][w]
    (nn/bgemm_uint8.py:89-114)."""

    @staticmethod
    def forward(ctx, x, w, lut, dx_lut, dw_lut):
        y, xq, wq = ops.bgemm_fake_uint8_claude_save(x, w, lut)
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


def bgemm_uint8_custom(x, w, lut, dx_lut, dw_lut):
    return _bgemm_uint8_custom.apply(x, w, lut, dx_lut, dw_lut)


class _bgemm_uint8(_bgemm_uint8_base):
    """Forward-only (nn/bgemm_uint8.py:117-127)."""

    @staticmethod
    def backward(ctx, grad_output):
        raise NotImplementedError(
            "bgemm_uint8 is forward-only; use bgemm_uint8_ste, "
            "bgemm_uint8_lre or bgemm_uint8_custom for training")


def bgemm_uint8(x, w, lut):
    return _bgemm_uint8.apply(x, w, lut)


# ------------------------------------------------------------- conv level
def _geom(x, geom):
    kernel_size, stride, padding, dilation, groups = geom
    if groups != 1:
        raise NotImplementedError(
            f"Conv2d_uint8 only supports groups=1 for now, got groups={groups}")
    return ops.conv_geom(tuple(x.shape), kernel_size, stride, padding, dilation)


class _conv2d_uint8_base(Function):
    """Forward of every conv-level uint8 Function: x is the quantized image
    (fp32 values 0..255), w [O, K] quantized values, zero_x the device scalar
    injected at out-of-image taps.  Returns the raw LUT sum [N, O, L]."""

    @staticmethod
    def _forward(ctx, x, w, lut, zero_x, geom):
        g = _geom(x, geom)
        y, wq = ops.conv_forward(x, w, lut, g, 0, 0, pad_dev=zero_x)
        ctx.g = g
        return y, wq


class _conv2d_uint8_ste(_conv2d_uint8_base):

    @staticmethod
    def forward(ctx, x, w, lut, zero_x, geom):
        y, wq = _conv2d_uint8_base._forward(ctx, x, w, lut, zero_x, geom)
        ctx.save_for_backward(x.detach().to(torch.uint8), wq, zero_x)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        xq, wq, zero_x = ctx.saved_tensors
        g = ctx.g
        ident = decode_table(xq.device, signed=False)
        go = grad_output.contiguous()
        grad_x = ops.conv_backward_data(go, wq, ident, g)
        grad_w = ops.conv_backward_weight(go, xq, ident, g, wq.size(0), 0, pad_dev=zero_x)
        return grad_x, grad_w, None, None, None


def conv2d_uint8_ste(x, w, lut, zero_x, geom):
    return _conv2d_uint8_ste.apply(x, w, lut, zero_x, geom)


class _conv2d_uint8_lre(_conv2d_uint8_base):

    @staticmethod
    def forward(ctx, x, w, lut, dx, dw, zero_x, geom):
        y, wq = _conv2d_uint8_base._forward(ctx, x, w, lut, zero_x, geom)
        ctx.save_for_backward(x.detach().to(torch.uint8), wq, zero_x)
        ctx.dx, ctx.dw = dx, dw
        return y

    @staticmethod
    def backward(ctx, grad_output):
        xq, wq, zero_x = ctx.saved_tensors
        g = ctx.g
        go = grad_output.contiguous()
        grad_x = ops.conv_backward_data(go, wq, ctx.dx.contiguous(), g)
        grad_w = ops.conv_backward_weight(go, xq, ctx.dw.contiguous(), g, wq.size(0), 0,
                                          pad_dev=zero_x)
        return grad_x, grad_w, None, None, None, None, None


def conv2d_uint8_lre(x, w, lut, dx, dw, zero_x, geom):
    return _conv2d_uint8_lre.apply(x, w, lut, dx, dw, zero_x, geom)


class _conv2d_uint8_custom(_conv2d_uint8_base):
    """Pair-table gradients of the uint8 conv: the forward's row-offset
    operand (padded taps at the device zero point z_x) is saved and read by
    the gradient kernels; the reference pads with z_x, unfolds and saves the
    uint8 index image (nn/Conv2d_uint8.py:283-294, nn/bgemm_uint8.py:89-114)."""

    @staticmethod
    def forward(ctx, x, w, lut, dx_lut, dw_lut, zero_x, geom):
        g = _geom(x, geom)
        y, wq, (xt, Rpad) = ops.conv_forward(x, w, lut, g, 0, 0, pad_dev=zero_x,
                                             return_operand=True)
        ctx.g, ctx.rpad = g, Rpad
        ctx.save_for_backward(xt, wq, dx_lut, dw_lut)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        xt, wq, dx_lut, dw_lut = ctx.saved_tensors
        g = ctx.g
        grad_col, grad_w = ops.custom_grads(
            (xt, ctx.rpad), wq, grad_output, dx_lut if ctx.needs_input_grad[0] else None,
            dw_lut if ctx.needs_input_grad[1] else None, g.N, g.C * g.KH * g.KW, g.OH * g.OW)
        grad_x = ops.col2im(grad_col, g) if grad_col is not None else None
        return grad_x, grad_w, None, None, None, None, None


def conv2d_uint8_custom(x, w, lut, dx_lut, dw_lut, zero_x, geom):
    return _conv2d_uint8_custom.apply(x, w, lut, dx_lut, dw_lut, zero_x, geom)


class _tap_sum(Function):
    """sum_k of the unfolded, z_x-padded image: [N, L]
    (xu.sum(dim=1) of nn/Conv2d_uint8.py:311)."""

    @staticmethod
    def forward(ctx, x, zero_x, geom):
        g = _geom(x, geom)
        ctx.g = g
        return ops.tap_sum(x, g, pad_dev=zero_x)

    @staticmethod
    def backward(ctx, grad_output):
        return ops.tap_sum_backward(grad_output, ctx.g), None, None


def tap_sum(x, zero_x, geom):
    return _tap_sum.apply(x, zero_x, geom)


# ---------------------------------------------------------- fused layer path
class _conv2d_uint8_fused(Function):
    """Conv2d_uint8's forward and backward as one Function: the composition of
    nn/Conv2d_uint8.py:257-325 (static fake-quant of x and W, the LUT conv of
    the raw uint8 values with z_x-padded taps, the zero-point correction
    y - z_w*sum_k q_x - z_x*sum_k q_w + K*z_x*z_w and the dequant by
    scale_x * scale_w), with no fp32 quantized image and no [N,O,L]
    temporaries:
      forward:  x -> uint8 image + mask, W -> uint8 GEMM operand + mask;
                implicit im2col LUT conv; the taps' sums of q_x (tap_sum) and
                sum_k q_w; one in-place pass for correction and dequant;
      backward: g' = go * (scale_x * scale_w[o]) feeds the estimator's
                gradient kernels (the custom kernels take the factor, no g'
                copy); the zero-point terms add -sum_o g' z_w[o] to every tap
                of a position (tap_sum's backward; folded with the STE into
                col2im on the custom path) and -z_x * sum_{n,l} g' to every
                tap of a channel; then the two fake-quant STEs.
    kind: 'ste' | 'lre' | 'custom'; tx / tw: the estimator's tables (STE:
    None, the identity decode table is used)."""

    @staticmethod
    def forward(ctx, x, weight, bias, scale_x, zero_x, scale_w, zero_w, lut, tx, tw, kind, geom,
                qmax_w):
        g = _geom(x, geom)
        O = weight.size(0)
        K = g.C * g.KH * g.KW
        _, mask_x, q8 = ops.fakequant_per_tensor(x, scale_x, 0, 255, zero_point=zero_x,
                                                  want_q=False, q8_dtype=torch.uint8)
        _, mask_w, wq, wt, Opad = ops.fakequant_per_channel(weight, scale_w, 0, qmax_w,
                                                            zero_point=zero_w, offset=0,
                                                            want_wt=True, want_q=False)
        # at most 16 weight indices (weight_bits <= 4): matrix-core LUT GEMM and grad_x
        wbase = 0 if qmax_w <= 15 else None
        xsum = ops.tap_sum(q8, g, pad_dev=zero_x)
        wsum = wq.sum(dim=1, dtype=torch.float32)
        b = None if bias is None else bias.detach().contiguous()
        # correction and dequant in the GEMM's epilogue (matrix-core path) or
        # as one in-place pass after it
        y, _, (xt, Rpad) = ops.conv_forward(
            q8, wq, lut, g, 0, 0, sx=scale_x.contiguous(), sw=scale_w.contiguous(), bias=b,
            pad_dev=zero_x, packed_w=(wq, wt, Opad), return_operand=True, wbase=wbase,
            u8=(xsum, wsum, zero_x.contiguous(), zero_w.contiguous()))
        ctx.save_for_backward(xt, mask_x, wq, mask_w.view(O, K), scale_x, zero_x, scale_w,
                              zero_w, tx, tw)
        ctx.g, ctx.rpad, ctx.kind = g, Rpad, kind
        ctx.has_bias, ctx.wshape = bias is not None, weight.shape
        ctx.wbase = wbase
        return y.view(g.N, O, g.OH, g.OW)

    @staticmethod
    def backward(ctx, grad_output):
        xt, mask_x, wq, mask_w, sx, zx, sw, zw, tx, tw = ctx.saved_tensors
        g = ctx.g
        O, K = wq.shape
        Lc = g.OH * g.OW
        go = grad_output.contiguous().view(g.N, O, Lc)
        c = (sx * sw).contiguous()          # d loss / d corrected sum = go * c[o]
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        need_b = ctx.has_bias and ctx.needs_input_grad[2]
        gx = gw = gb = None
        # zero-point terms: -sum_o g' z_w[o] per position (a channel reduction
        # per image) and -z_x sum_{n,l} g' per channel
        gxs = gsum = None
        if (need_w or need_b) and O <= ops.ZERO_POINT_SUM_MAX_O:
            gxs, gsum = ops.zero_point_terms(go, sx, sw, zw, want_pos=need_x)
        else:
            gxs = ops.zero_point_pos(go, sx, sw, zw) if need_x else None
            gsum = go.sum(dim=(0, 2)) if (need_w or need_b) else None
        if ctx.kind == 'custom':
            # a 1x1 stride-1 unpadded conv's column gradient is its image
            # gradient: the matrix-core grad_x applies the zero-point term and
            # the STE in its epilogue (the fold's operations for that geometry)
            pointwise = (ctx.wbase is not None and need_x and g.KH == 1 and g.KW == 1 and
                         g.SH == 1 and g.SW == 1 and g.PH == 0 and g.PW == 0)
            # the weight zero-point term and the weight STE in grad_w's slice sum
            fuse_w = need_w and gsum is not None
            grad_col, gw_q = ops.custom_grads(
                (xt, ctx.rpad), wq, go, tx if need_x else None, tw if need_w else None, g.N,
                K, Lc, wbase=ctx.wbase, dy_scale=c,
                img_ste=(gxs, mask_x, sx) if pointwise else None,
                mask_w=mask_w if fuse_w else None, scale_w=sw if fuse_w else None,
                w_zero_point=(gsum, sx, zx) if fuse_w else None)
            if fuse_w:
                gw = gw_q.view(ctx.wshape)
                need_w = False
            if pointwise:
                gx = grad_col.view(mask_x.shape)
            elif need_x:   # fold, zero-point term and the STE in one pass
                gx = ops.col2im(grad_col, g, pos=gxs, mask=mask_x, scale=sx)
        else:
            gp = go * c.view(1, -1, 1)
            if ctx.kind == 'ste':
                tx = tw = decode_table(gp.device, signed=False)
            gw_q = ops.conv_backward_weight_rows(gp, (xt, ctx.rpad), tw.contiguous(), g, O) \
                if need_w else None
            if need_x:
                grad_q = ops.conv_backward_data(gp, wq, tx.contiguous(), g)
                grad_q += ops.tap_sum_backward(gxs, g)
                gx = ops.fakequant_per_tensor_backward(grad_q, mask_x, sx)
        if need_w:
            gw_q -= (gsum * c).mul_(zx).view(-1, 1)
            gw = ops.fakequant_per_tensor_backward(gw_q, mask_w, sw, channels=O,
                                                   inner=K).view(ctx.wshape)
        if need_b:
            gb = gsum
        return gx, gw, gb, None, None, None, None, None, None, None, None, None, None


def conv2d_uint8_fused(x, weight, bias, scale_x, zero_x, scale_w, zero_w, lut, tx, tw, kind,
                       geom, qmax_w):
    return _conv2d_uint8_fused.apply(x, weight, bias, scale_x, zero_x, scale_w, zero_w, lut, tx,
                                     tw, kind, geom, qmax_w)
