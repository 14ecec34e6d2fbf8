"""Conv2d_int8: int8 approximate-multiplier convolution (decoupled: integer
LUT conv + dequant at the end).  Mirrors approxtorch/nn/Conv2d_int8.py:9-220:
same constructor, buffers (lut, scale_x, scale_w, dx, dw), EMA rules and
forward composition; the per-step statistics, fake-quant and LUT conv run as
HIP kernels.
"""
import math

import torch
import torch.distributed as dist
import torch.nn as nn
from torch.nn.modules.utils import _pair

from . import bgemm_int8, quantization
from ..backend import _lib as L
from ..backend import ops


def _check_stat_inputs(x, *buffers, lowp=False):
    """The kernels behind the statistic updates read x as fp32 device memory
    (fp16 / bf16 as well with lowp: the *_dt kernels) and write the fp32
    scale buffers in place: check both before any launch (the reference's
    ops reject the same inputs, csrc/claude/quantization.cu:190-193)."""
    if lowp:
        ops.require_cuda_float(x, "x")
    else:
        ops.require_cuda_f32(x, "x")
    for name, b in buffers:
        if not b.is_cuda or b.device != x.device or b.dtype != torch.float32:
            raise RuntimeError(f"buffer {name} must be a float32 CUDA tensor on {x.device}; "
                               f"move the layer to the input's device first")


def _bump(*buffers):
    """The EMA kernels write the buffers through raw pointers; bump their
    version counters as torch's in-place copy_() in the reference does, so a
    backward that saved an earlier value raises instead of reading the new one."""
    for b in buffers:
        torch.autograd.graph.increment_version(b)


def _ema_coeffs(m):
    # torch evaluates `m * cur + (1 - m) * old` with both python scalars cast
    # to fp32: reproduce those two constants exactly.
    return float(torch.tensor(m, dtype=torch.float32)), \
        float(torch.tensor(1 - m, dtype=torch.float32))


class Conv2d_int8(nn.Module):
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
                 weight_bits: int = 8,
                 save_image: bool = False):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        if groups != 1 and not (groups == in_channels and out_channels == in_channels):
            raise NotImplementedError(
                "Conv2d_int8 supports groups=1 or depthwise "
                f"(groups == in_channels == out_channels), got groups={groups}, "
                f"in={in_channels}, out={out_channels}")
        self.groups = groups
        if grad not in ('ste', 'lre', 'custom'):
            raise ValueError(f"grad must be 'ste', 'lre' or 'custom', got {grad}")
        if grad == 'custom' and groups != 1:
            raise NotImplementedError("custom gradient currently supports only groups=1")
        self.grad = grad
        self.qmin = -127
        self.qmax = 127
        self.weight_bits = weight_bits
        if not 3 <= weight_bits <= 8:
            raise ValueError(f"weight_bits must be between 3 and 8, got {weight_bits}")
        if not 0.0 <= scale_momentum <= 1.0:
            raise ValueError(f"scale_momentum must be between 0 and 1, got {scale_momentum}")
        self.scale_momentum = scale_momentum
        self.update_scale = update_scale
        # No counterpart in the reference's constructor (an added keyword):
        # False keeps the forward's row-offset operand (uint16 per unfolded
        # tap) for grad_w; True keeps the int8 image instead (1 byte per
        # input element, the reference's saved tensor) and grad_w unfolds it
        # again in its loads (atx_conv_bwd_weight): less memory, slower
        # backward.
        self.save_image = save_image

        self.register_buffer('lut', lut)
        self.weight = nn.Parameter(torch.empty(self.out_channels,
                                               self.in_channels // self.groups,
                                               self.kernel_size[0], self.kernel_size[1]))
        self.register_buffer('scale_x', torch.tensor(1.0))
        self.register_buffer('scale_w', torch.ones(self.out_channels))

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
            self.register_buffer('dx', dx)
            self.register_buffer('dw', dw)
        elif grad == 'custom':
            if dx is None or dw is None:
                raise ValueError("dx and dw are required when grad='custom'")
            if not isinstance(dx, torch.Tensor) or not isinstance(dw, torch.Tensor):
                raise TypeError("custom dx and dw must be torch.Tensor objects")
            if dx.numel() != 256 * 256 or dw.numel() != 256 * 256:
                raise ValueError("custom dx and dw must each have 65536 elements "
                                 "for grad_lut[x + 128][w + 128]")
            if dx.dtype != torch.float32 or dw.dtype != torch.float32:
                raise TypeError("custom dx and dw must have dtype torch.float32")
            self.register_buffer('dx', dx.contiguous().view(-1))
            self.register_buffer('dw', dw.contiguous().view(-1))

    def reset_parameters(self):
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            fan_in = (self.in_channels // self.groups) * self.kernel_size[0] * self.kernel_size[1]
            bound = 1 / math.sqrt(fan_in) if fan_in > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

    def __repr__(self):
        return (f"Conv2d_int8(in_channels={self.in_channels}, out_channels={self.out_channels}, "
                f"kernel_size={self.kernel_size}, stride={self.stride}, padding={self.padding}, "
                f"dilation={self.dilation}, groups={self.groups}, grad={self.grad}, "
                f"weight_bits={self.weight_bits})")

    def unfreeze_scale(self):
        self.update_scale = True

    def freeze_scale(self):
        self.update_scale = False

    def _update_scale(self, x):
        """scale_x <- m * absmax(x)/127 + (1-m) * scale_x (nn/Conv2d_int8.py:137-146).
        The absmax reduction and the EMA run on the device; under DDP the
        statistic is MAX-all-reduced in between so every rank's scale agrees.
        Returns a device int32 flag, set when x >= 0 everywhere (the LUT GEMM
        of this forward may then build half-height tables), or None.  x >= 0
        means every quantized x >= 0 only because the fake-quant divides by
        max(scale_x, 1e-12) > 0 (whatever scale_x holds) and qmax >= 0;
        conv2d_int8_fused checks the latter."""
        _check_stat_inputs(x, ("scale_x", self.scale_x), lowp=True)
        with torch.no_grad():
            xc = x.contiguous()
            stat = torch.empty((), dtype=torch.float32, device=x.device)
            ws = ops._reduce_ws(x.device)
            s = L.stream_of(xc)
            m32, om32 = _ema_coeffs(self.scale_momentum)
            denom = float((self.qmax - self.qmin) / 2)
            upper = None
            # an fp16 / bf16 x: abs_max and the first EMA terms are that dtype's
            dt = ops.dtype_code(xc)
            if not (dist.is_available() and dist.is_initialized()):
                # no all-reduce in between: the EMA runs in the reduction's last launch
                upper = torch.empty((), dtype=torch.int32, device=x.device)
                L.call("atx_absmax_ema_upper_dt", L.ptr(xc), dt, xc.numel(), L.ptr(ws),
                       L.ptr(stat), denom, m32, om32, L.ptr(self.scale_x), L.ptr(upper), s)
            else:
                L.call("atx_absmax_dt", L.ptr(xc), dt, xc.numel(), L.ptr(ws), L.ptr(stat), s)
                dist.all_reduce(stat, op=dist.ReduceOp.MAX)
                L.call("atx_ema_absmax_apply_dt", L.ptr(stat), dt, denom, m32, om32,
                       L.ptr(self.scale_x), s)
        _bump(self.scale_x)
        return upper

    def _update_scale_w(self):
        """Per-channel EMA of absmax(W)/qmax_w; zero channels keep their scale
        (nn/Conv2d_int8.py:148-158)."""
        _check_stat_inputs(self.weight, ("scale_w", self.scale_w), lowp=True)
        with torch.no_grad():
            w = self.weight.detach().contiguous()
            O = w.size(0)
            m32, om32 = _ema_coeffs(self.scale_momentum)
            L.call("atx_weight_scale_ema_dt", L.ptr(w), ops.dtype_code(w), O,
                   w.numel() // max(O, 1), float(2 ** (self.weight_bits - 1) - 1), m32, om32, 0,
                   L.ptr(self.scale_w), L.stream_of(w))
        _bump(self.scale_w)

    def reset_weight_qparams(self):
        """scale_w = absmax(W)/qmax_w per channel (1 for zero channels); runs at
        construction / conversion time, possibly on the CPU
        (nn/Conv2d_int8.py:160-167)."""
        with torch.no_grad():
            qmax_w = 2 ** (self.weight_bits - 1) - 1
            w = self.weight.detach()
            if w.is_cuda:
                _check_stat_inputs(w, ("scale_w", self.scale_w), lowp=True)
                wc = w.contiguous()
                O = wc.size(0)
                L.call("atx_weight_scale_ema_dt", L.ptr(wc), ops.dtype_code(wc), O,
                       wc.numel() // max(O, 1), float(qmax_w), 1.0, 0.0, 1,
                       L.ptr(self.scale_w), L.stream_of(wc))
                _bump(self.scale_w)
                return
            absmax = w.abs().amax(dim=tuple(range(1, w.dim())))
            self.scale_w.copy_(torch.where(absmax > 0, absmax / qmax_w, torch.ones_like(absmax)))

    def forward(self, x: torch.Tensor):
        B, _, H, W = x.shape
        O, _, kH, kW = self.weight.shape
        sH, sW = self.stride
        pH, pW = self.padding
        dH, dW = self.dilation
        OH = (H + 2 * pH - dH * (kH - 1) - 1) // sH + 1
        OW = (W + 2 * pW - dW * (kW - 1) - 1) // sW + 1

        upper = None
        if self.training and self.update_scale:
            upper = self._update_scale(x)
            self._update_scale_w()

        qmax_w = 2 ** (self.weight_bits - 1) - 1
        geom = ((kH, kW), self.stride, self.padding, self.dilation, self.groups)
        if self.grad in ('ste', 'lre'):
            # fake-quant, LUT conv and dequant in one Function (same values and
            # gradients as the composition below, without the fp32 fake-quantized
            # tensors)
            if self.grad == 'lre':
                tx, tw = self.dx, self.dw
            else:
                tx = tw = bgemm_int8.decode_table(x.device)
            return bgemm_int8.conv2d_int8_fused(x, self.weight, self.bias, self.scale_x,
                                                self.scale_w, self.lut, tx, tw, geom,
                                                self.qmin, self.qmax, qmax_w, x_upper=upper,
                                                save_image=getattr(self, "save_image", False))

        x = quantization.static_quantize_int8(x, self.scale_x, self.qmin, self.qmax)
        w = quantization.static_quantize_int8(self.weight, self.scale_w, -qmax_w, qmax_w,
                                              ch_axis=0)
        s_w = self.scale_w

        if self.grad == 'lre':
            y = bgemm_int8.conv2d_int8_lre(x, w.view(O, -1), self.lut, self.dx, self.dw, geom)
        elif self.grad == 'custom':
            y = bgemm_int8.conv2d_int8_custom(x, w.view(O, -1), self.lut, self.dx, self.dw,
                                              geom, qmax_w)
        else:
            y = bgemm_int8.conv2d_int8_ste(x, w.view(O, -1), self.lut, geom)

        y = y.view(B, O, OH, OW)
        s = (self.scale_x * s_w).view(1, -1, 1, 1)
        if self.bias is not None:
            y = torch.addcmul(self.bias.view(1, -1, 1, 1), y, s)
        else:
            y = y * s
        return y
