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
           "conv2d_uint8_ste", "conv2d_uint8_lre", "conv2d_uint8_custom", "tap_sum"]


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
