"""Conv2d_uint8: uint8 x uint8 approximate-multiplier convolution with static
asymmetric quantization (per-tensor activations, per-channel weights).
Mirrors approxtorch/nn/Conv2d_uint8.py:11-325: same buffers (x_min, x_max,
w_min, w_max, scale_x, zero_x, scale_w, zero_w, lut, dx, dw), legacy
checkpoint loading and the differentiable zero-point correction

  sum_k (q_x - z_x)(q_w - z_w) = LUTSUM - z_w*sum_k q_x - z_x*sum_k q_w + K*z_x*z_w.

Extension: `weight_bits` (default 8, the reference's only setting) quantizes
weights to [0, 2**weight_bits - 1] with per-channel EMA qparams.
"""
import math

import torch
import torch.distributed as dist
import torch.nn as nn
from torch.nn.modules.utils import _pair

from . import bgemm_uint8
from ..backend import _lib as L
from ..backend import ops
from .Conv2d_int8 import _bump, _check_stat_inputs, _ema_coeffs


def uint8_qparams(mn, mx, qmax=255):
    """(scale, zero_point) from min/max statistics, range clamped to include 0
    (nn/Conv2d_uint8.py:11-23)."""
    mn = torch.clamp(mn, max=0.0)
    mx = torch.clamp(mx, min=0.0)
    scale = torch.clamp((mx - mn) / qmax, min=1e-12)
    zero = torch.round(-mn / scale).clamp(0.0, float(qmax))
    return scale, zero


class Conv2d_uint8(nn.Module):
    # buffers that alias tables owned by the caller (never moved or copied
    # when the layer adopts another layer's device)
    caller_tables = ("lut", "dx", "dw")

    def __init__(self,
                 in_channels: int,
                 out_channels: int,
                 kernel_size,
                 lut: torch.Tensor,
                 grad: str = 'ste',
                 dx: torch.Tensor | None = None,
                 dw: torch.Tensor | None = None,
                 bias=None,
                 stride=1,
                 padding=0,
                 dilation=1,
                 groups: int = 1,
                 update_scale: bool = True,
                 scale_momentum: float = 0.05,
                 weight_bits: int = 8):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        if groups != 1:
            raise NotImplementedError(
                f"Conv2d_uint8 only supports groups=1 for now, got groups={groups}")
        self.groups = groups
        if grad not in ('ste', 'lre', 'custom'):
            raise ValueError(f"grad must be 'ste', 'lre' or 'custom', got {grad}")
        self.grad = grad
        self.qmin = 0
        self.qmax = 255
        if not 1 <= weight_bits <= 8:
            raise ValueError(f"weight_bits must be between 1 and 8, got {weight_bits}")
        self.weight_bits = weight_bits
        self.qmax_w = 2 ** weight_bits - 1
        if not 0.0 <= scale_momentum <= 1.0:
            raise ValueError(f"scale_momentum must be between 0 and 1, got {scale_momentum}")
        self.scale_momentum = scale_momentum
        self.update_scale = update_scale

        self.register_buffer('lut', lut)
        self.weight = nn.Parameter(torch.empty(self.out_channels, self.in_channels,
                                               self.kernel_size[0], self.kernel_size[1]))
        self.register_buffer('x_min', torch.tensor(0.0))
        self.register_buffer('x_max', torch.tensor(1.0))
        self.register_buffer('w_min', torch.zeros(self.out_channels))
        self.register_buffer('w_max', torch.ones(self.out_channels))
        self.register_buffer('scale_x', torch.tensor(1.0 / self.qmax))
        self.register_buffer('zero_x', torch.tensor(0.0))
        self.register_buffer('scale_w', torch.ones(self.out_channels))
        self.register_buffer('zero_w', torch.zeros(self.out_channels))

        if isinstance(bias, torch.Tensor) or bias is True:
            self.bias = nn.Parameter(torch.empty(self.out_channels))
        elif bias is False or bias is None:
            self.bias = None
        else:
            raise ValueError("Invalid bias type")

        self.reset_parameters()
        self.reset_weight_qparams()

        if isinstance(bias, torch.Tensor):
            if bias.shape != (self.out_channels,):
                raise ValueError(
                    f"bias must have shape ({self.out_channels},), got {tuple(bias.shape)}")
            with torch.no_grad():
                self.bias.copy_(bias)

        if grad == 'lre':
            if dx is None or dw is None:
                raise ValueError("dx and dw are required when grad='lre'")
            if not isinstance(dx, torch.Tensor) or not isinstance(dw, torch.Tensor):
                raise TypeError("lre dx and dw must be torch.Tensor objects")
            if dx.numel() != 256 or dw.numel() != 256:
                raise ValueError("lre dx and dw must each have 256 elements, indexed by "
                                 "the raw uint8 operand value")
            if dx.dtype != torch.float32 or dw.dtype != torch.float32:
                raise TypeError("lre dx and dw must have dtype torch.float32")
            self.register_buffer('dx', dx.contiguous().view(-1))
            self.register_buffer('dw', dw.contiguous().view(-1))
        elif grad == 'custom':
            if dx is None or dw is None:
                raise ValueError("dx and dw are required when grad='custom'")
            if not isinstance(dx, torch.Tensor) or not isinstance(dw, torch.Tensor):
                raise TypeError("custom dx and dw must be torch.Tensor objects")
            if dx.numel() != 256 * 256 or dw.numel() != 256 * 256:
                raise ValueError("custom dx and dw must each have 65536 elements for "
                                 "grad_lut[x][w]")
            if dx.dtype != torch.float32 or dw.dtype != torch.float32:
                raise TypeError("custom dx and dw must have dtype torch.float32")
            self.register_buffer('dx', dx.contiguous().view(-1))
            self.register_buffer('dw', dw.contiguous().view(-1))

    def reset_parameters(self):
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            fan_in = self.in_channels * self.kernel_size[0] * self.kernel_size[1]
            bound = 1 / math.sqrt(fan_in) if fan_in > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

    def __repr__(self):
        extra = f", weight_bits={self.weight_bits}" if self.weight_bits != 8 else ""
        return (f"Conv2d_uint8(in_channels={self.in_channels}, out_channels={self.out_channels}, "
                f"kernel_size={self.kernel_size}, stride={self.stride}, padding={self.padding}, "
                f"dilation={self.dilation}, groups={self.groups}, grad={self.grad}{extra})")

    def unfreeze_scale(self):
        self.update_scale = True

    def freeze_scale(self):
        self.update_scale = False

    def reset_weight_qparams(self):
        """w_min / w_max from the current weight (per output channel), then
        every qparam from the statistics."""
        with torch.no_grad():
            w = self.weight.detach()
            dims = tuple(range(1, w.dim()))
            self.w_min.copy_(w.amin(dim=dims))
            self.w_max.copy_(w.amax(dim=dims))
        self._reset_qparams_from_stats()

    def _reset_qparams_from_stats(self):
        with torch.no_grad():
            scale_x, zero_x = uint8_qparams(self.x_min, self.x_max, self.qmax)
            scale_w, zero_w = uint8_qparams(self.w_min, self.w_max, self.qmax_w)
            self.scale_x.copy_(scale_x)
            self.zero_x.copy_(zero_x)
            self.scale_w.copy_(scale_w)
            self.zero_w.copy_(zero_w)

    # Checkpoint compatibility (nn/Conv2d_uint8.py:195-223): a checkpoint
    # holding only the min/max statistics gets its qparams derived from them
    # (and they are not reported missing); a stored zero point must be an
    # integer inside its quantized range.
    _QPARAM_FIELDS = ('scale_x', 'zero_x', 'scale_w', 'zero_w')

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict,
                              missing_keys, unexpected_keys, error_msgs):
        qparam_keys = {prefix + f for f in self._QPARAM_FIELDS}
        derive = qparam_keys.isdisjoint(state_dict.keys())
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict,
                                      missing_keys, unexpected_keys, error_msgs)
        if derive:
            self._reset_qparams_from_stats()
            missing_keys[:] = [k for k in missing_keys if k not in qparam_keys]
        for field, top in (('zero_x', self.qmax), ('zero_w', self.qmax_w)):
            z = getattr(self, field)
            # NaN fails z == round(z); +-inf fails the range
            if not bool(torch.all((z == torch.round(z)) & (z >= self.qmin) & (z <= top))):
                error_msgs.append(f"{prefix}{field} must contain integer-valued "
                                  f"values in [{self.qmin}, {top}]")

    def _update_scale(self, x):
        """min/max EMA of the activations, then qparams, on the device; MIN/MAX
        all-reduce under DDP (nn/Conv2d_uint8.py:225-240)."""
        _check_stat_inputs(x, ("x_min", self.x_min), ("x_max", self.x_max),
                           ("scale_x", self.scale_x), ("zero_x", self.zero_x))
        with torch.no_grad():
            xc = x.contiguous()
            mn = torch.empty((), dtype=torch.float32, device=x.device)
            mx = torch.empty((), dtype=torch.float32, device=x.device)
            ws = ops._reduce_ws(x.device)
            s = L.stream_of(xc)
            m32, om32 = _ema_coeffs(self.scale_momentum)
            if not (dist.is_available() and dist.is_initialized()):
                # no all-reduce in between: the EMA runs in the reduction's last launch
                L.call("atx_minmax_ema", L.ptr(xc), xc.numel(), L.ptr(ws), L.ptr(mn),
                       L.ptr(mx), m32, om32, self.qmax, L.ptr(self.x_min), L.ptr(self.x_max),
                       L.ptr(self.scale_x), L.ptr(self.zero_x), s)
            else:
                L.call("atx_minmax", L.ptr(xc), xc.numel(), L.ptr(ws), L.ptr(mn), L.ptr(mx), s)
                dist.all_reduce(mn, op=dist.ReduceOp.MIN)
                dist.all_reduce(mx, op=dist.ReduceOp.MAX)
                L.call("atx_ema_minmax_apply", L.ptr(mn), L.ptr(mx), m32, om32, self.qmax,
                       L.ptr(self.x_min), L.ptr(self.x_max), L.ptr(self.scale_x),
                       L.ptr(self.zero_x), s)
        _bump(self.x_min, self.x_max, self.scale_x, self.zero_x)

    def _update_scale_w(self):
        """Per-channel min/max EMA of the weights + qparams (nn/Conv2d_uint8.py:242-255)."""
        _check_stat_inputs(self.weight, ("w_min", self.w_min), ("w_max", self.w_max),
                           ("scale_w", self.scale_w), ("zero_w", self.zero_w))
        with torch.no_grad():
            w = self.weight.detach().contiguous()
            O = w.size(0)
            m32, om32 = _ema_coeffs(self.scale_momentum)
            L.call("atx_weight_minmax_ema", L.ptr(w), O, w.numel() // max(O, 1), m32, om32,
                   self.qmax_w, L.ptr(self.w_min), L.ptr(self.w_max), L.ptr(self.scale_w),
                   L.ptr(self.zero_w), L.stream_of(w))
        _bump(self.w_min, self.w_max, self.scale_w, self.zero_w)

    def forward(self, x: torch.Tensor):
        # the uint8 layer's kernels read fp32 activations and weights only
        ops.require_cuda_f32(x, "x")
        ops.require_cuda_f32(self.weight, "weight")
        kH, kW = self.weight.shape[2:]
        if self.training and self.update_scale:
            self._update_scale(x)
            self._update_scale_w()

        # fake-quant, LUT conv, zero-point correction and dequant in one
        # Function (the composition of nn/Conv2d_uint8.py:257-325, with the
        # same values and gradients; see bgemm_uint8._conv2d_uint8_fused)
        geom = ((kH, kW), self.stride, self.padding, self.dilation, self.groups)
        tx, tw = (self.dx, self.dw) if self.grad in ('lre', 'custom') else (None, None)
        return bgemm_uint8.conv2d_uint8_fused(x, self.weight, self.bias, self.scale_x,
                                              self.zero_x, self.scale_w, self.zero_w, self.lut,
                                              tx, tw, self.grad, geom, self.qmax_w)
