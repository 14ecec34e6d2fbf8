"""Static fake-quant (returns integer-valued q; the caller dequantizes).

  int8 symmetric     q = clamp(round(x/s),     qmin, qmax)   default [-127, 127]
  uint8 asymmetric   q = clamp(round(x/s + z), qmin, qmax)   default [0, 255]

per-tensor (ch_axis=None) or per-channel (ch_axis=int).  STE backward:
gx = go * mask / s with mask = qmin <= x/s (+z) <= qmax on the pre-round value.

Mirrors approxtorch/nn/quantization.py:37-191.  Every path runs the fused
HIP kernels (atx_fakequant_*); tensors must live on the GPU and be fp32,
fp16 or bf16.  An fp16 / bf16 x gets torch's semantics for the reference's
statements: with 0-dim scale (and zero point) the per-tensor v = x / s is
computed in x's dtype and q keeps it (atx_fakequant_fwd_dt); a per-channel
or 1-element (1-dim) scale promotes x / s, and q, to fp32, which the fp32
kernels compute from x's exact fp32 value.
"""
import torch
from torch.autograd import Function

from ..backend import ops


def _require_gpu_float(x, name="x"):
    if not x.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (approxtorch_amd runs on the GPU)")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"{name} must be float32, float16 or bfloat16, got {x.dtype}")


def _promoted(x, scale, zero_point=None):
    """x as the fp32 kernels must read it: a low-precision x stays in its
    dtype only when torch would compute x / s (+ z) in it, i.e. with 0-dim
    scale and zero point; a dimensioned scale promotes the statements to
    fp32 (x converted exactly).  A 0-dim scale with a dimensioned zero point
    (fp32 added to a low-precision quotient) is not supported."""
    if x.dtype == torch.float32:
        return x
    if scale.dim() > 0:
        return x.float()
    if zero_point is not None and zero_point.dim() > 0:
        raise NotImplementedError(
            "fp16/bf16 fake-quant with a 0-dim scale needs a 0-dim zero_point")
    return x


def _param(p, x):
    # python number -> fp32 scalar tensor on x's device (nn/quantization.py:138-143)
    if isinstance(p, torch.Tensor):
        return p
    return torch.tensor(float(p), dtype=torch.float32, device=x.device)


def _as_f32(p, x):
    p = _param(p, x)
    if p.dtype != torch.float32 or p.device != x.device:
        p = p.to(device=x.device, dtype=torch.float32)
    return p.contiguous()


class _static_quantize_per_tensor_symmetric(Function):

    @staticmethod
    def forward(ctx, x, scale, qmin, qmax):
        q, mask, _ = ops.fakequant_per_tensor(x, scale, qmin, qmax)
        ctx.save_for_backward(mask, scale)
        return q

    @staticmethod
    def backward(ctx, grad_output):
        mask, s = ctx.saved_tensors
        return ops.fakequant_per_tensor_backward(grad_output, mask, s), None, None, None


class _static_quantize_per_tensor_asymmetric(Function):

    @staticmethod
    def forward(ctx, x, scale, zero_point, qmin, qmax):
        q, mask, _ = ops.fakequant_per_tensor(x, scale, qmin, qmax, zero_point=zero_point)
        ctx.save_for_backward(mask, scale)
        return q

    @staticmethod
    def backward(ctx, grad_output):
        # zero_point is additive: dq/dx = mask / s, as in the symmetric case
        mask, s = ctx.saved_tensors
        return (ops.fakequant_per_tensor_backward(grad_output, mask, s),
                None, None, None, None)


def _channel_first(x, ch_axis):
    return x if ch_axis == 0 else x.movedim(ch_axis, 0).contiguous()


class _static_quantize_per_channel(Function):

    @staticmethod
    def forward(ctx, x, scale, zero_point, ch_axis, qmin, qmax):
        xf = _channel_first(x, ch_axis)
        q, mask, _, _, _ = ops.fakequant_per_channel(xf, scale, qmin, qmax, zero_point)
        ctx.save_for_backward(mask, scale)
        ctx.ch_axis = ch_axis
        ctx.shape0 = xf.shape
        return q if ch_axis == 0 else q.movedim(0, ch_axis)

    @staticmethod
    def backward(ctx, grad_output):
        mask, s = ctx.saved_tensors
        go = _channel_first(grad_output, ctx.ch_axis)
        C = go.size(0)
        gx = ops.fakequant_per_tensor_backward(go, mask, s, channels=C,
                                               inner=max(go.numel() // max(C, 1), 1))
        if ctx.ch_axis != 0:
            gx = gx.movedim(0, ctx.ch_axis)
        return gx, None, None, None, None, None


def _check_per_channel_param(name, p, x, ch_axis):
    if p.numel() != x.shape[ch_axis]:
        raise ValueError(
            f"per-channel {name} must have {x.shape[ch_axis]} elements "
            f"(= x.shape[{ch_axis}]), got {p.numel()}")


def static_quantize_int8(x, scale, qmin=-127, qmax=127, ch_axis=None):
    """int8 symmetric static fake-quant: q = clamp(round(x/scale), qmin, qmax).

    scale: per-tensor scalar (1-element tensor or number) or, with ch_axis,
    a [x.shape[ch_axis]] tensor.  Returns q as an fp32 integer-valued tensor.
    nn/quantization.py:153-171."""
    if qmin >= qmax:
        raise ValueError(f"qmin must be < qmax, got [{qmin}, {qmax}]")
    _require_gpu_float(x)
    scale = _as_f32(scale, x)
    if ch_axis is None:
        return _static_quantize_per_tensor_symmetric.apply(_promoted(x, scale), scale, qmin,
                                                           qmax)
    _check_per_channel_param('scale', scale, x, ch_axis)
    return _static_quantize_per_channel.apply(x.float(), scale, None, ch_axis, qmin, qmax)


def static_quantize_uint8(x, scale, zero_point, qmin=0, qmax=255, ch_axis=None):
    """uint8 asymmetric static fake-quant: q = clamp(round(x/scale + zero_point),
    qmin, qmax).  nn/quantization.py:174-191."""
    if qmin >= qmax:
        raise ValueError(f"qmin must be < qmax, got [{qmin}, {qmax}]")
    _require_gpu_float(x)
    scale = _as_f32(scale, x)
    zero_point = _as_f32(zero_point, x)
    if ch_axis is None:
        return _static_quantize_per_tensor_asymmetric.apply(_promoted(x, scale, zero_point),
                                                            scale, zero_point, qmin, qmax)
    _check_per_channel_param('scale', scale, x, ch_axis)
    _check_per_channel_param('zero_point', zero_point, x, ch_axis)
    return _static_quantize_per_channel.apply(x.float(), scale, zero_point, ch_axis, qmin,
                                              qmax)
