"""PyTorch-CPU restatement of the LUT conv layers — TEST INFRASTRUCTURE and
the timed CPU baseline of bench.py (never part of the product path).

Forward (nn/Conv2d_int8.py:171-220, nn/Conv2d_uint8.py:257-325 semantics):
fake-quant -> F.unfold -> int64 LUT index -> lut.take -> int64 sum over K
(chunked over L to bound memory) -> dequant.  Backward: the estimator math
of nn/bgemm_int8.py / nn/bgemm_uint8.py written with torch-CPU ops (STE /
LRE as dense products of mapped operands, custom as pair-table gathers).
"""
import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.autograd import Function

_CHUNK = 1 << 22     # index elements per chunk


def _fq(x, s, qmin, qmax, z=None):
    s = torch.clamp(s, min=1e-12)
    v = x / s if z is None else x / s + z
    mask = (v >= qmin) & (v <= qmax)
    return torch.clamp(torch.round(v), qmin, qmax), mask


class _FQ(Function):
    @staticmethod
    def forward(ctx, x, s, qmin, qmax, z):
        q, m = _fq(x, s, qmin, qmax, z)
        ctx.save_for_backward(m, torch.clamp(s, min=1e-12))
        return q

    @staticmethod
    def backward(ctx, g):
        m, s = ctx.saved_tensors
        return g * m.to(g.dtype) / s, None, None, None, None


def lut_sum(xi, wi, lut):
    """int64 sum_k lut[xi*256 + wi]: xi [N,K,L] int64 index, wi [O,K]."""
    N, K, L = xi.shape
    O = wi.shape[0]
    y = torch.empty(N, O, L, dtype=torch.int64)
    step = max(1, _CHUNK // max(1, K * O))
    lut = lut.reshape(-1).to(torch.int64)
    for n in range(N):
        for l0 in range(0, L, step):
            idx = xi[n, :, None, l0:l0 + step] * 256 + wi.t()[:, :, None]   # [K, O, l]
            y[n, :, l0:l0 + step] = lut.take(idx).sum(dim=0)
    return y


class _LUTConv(Function):
    """y = LUT sum of the quantized image/weights; backward per estimator."""

    @staticmethod
    def forward(ctx, qx, qw, lut, geom, offset, pad, kind, tx, tw):
        k, s, p, d = geom
        N, C, H, W = qx.shape
        xp = F.pad(qx - pad, (p[1], p[1], p[0], p[0])) + pad
        xu = F.unfold(xp, k, dilation=d, padding=0, stride=s)            # [N, K, L]
        xi = (xu.round().to(torch.int64) + offset).clamp(0, 255)
        wi = (qw.reshape(qw.shape[0], -1).round().to(torch.int64) + offset).clamp(0, 255)
        y = lut_sum(xi, wi, lut).to(torch.float32)
        ctx.save_for_backward(xi, wi)
        ctx.meta = (qx.shape, qw.shape, geom, offset, kind, tx, tw)
        return y

    @staticmethod
    def backward(ctx, go):
        xi, wi = ctx.saved_tensors
        xshape, wshape, (k, s, p, d), offset, kind, tx, tw = ctx.meta
        if kind in ("ste", "lre"):
            if kind == "ste":
                tx = tw = torch.arange(256, dtype=torch.float32) - offset
            gcol = torch.einsum("nol,ok->nkl", go, tx[wi])
            gw = torch.einsum("nol,nkl->ok", go, tw[xi])
        else:
            dxl, dwl = tx.reshape(256, 256), tw.reshape(256, 256)
            gcol = torch.zeros(xi.shape)
            gw = torch.zeros(wi.shape)
            for o in range(wi.shape[0]):
                gcol += go[:, o, None, :] * dxl[xi, wi[o][None, :, None]]
                gw[o] = (go[:, o, None, :] * dwl[xi, wi[o][None, :, None]]).sum(dim=(0, 2))
        N, C, H, W = xshape
        gpad = F.fold(gcol, (H + 2 * p[0], W + 2 * p[1]), k, dilation=d, padding=0, stride=s)
        gx = gpad[:, :, p[0]:p[0] + H, p[1]:p[1] + W]
        return gx, gw.reshape(wshape), None, None, None, None, None, None, None


class LUTConv2dCPU(nn.Module):
    """CPU twin of Conv2d_int8 / Conv2d_uint8 (given qparams; EMA rules as the
    reference, evaluated with torch-CPU ops)."""

    def __init__(self, layer):
        super().__init__()
        self.qtype = "uint8" if hasattr(layer, "zero_x") else "int8"
        self.weight = nn.Parameter(layer.weight.detach().cpu().clone())
        self.bias = None if layer.bias is None else nn.Parameter(layer.bias.detach().cpu().clone())
        for name in ("lut", "scale_x", "scale_w", "zero_x", "zero_w", "x_min", "x_max", "w_min",
                     "w_max", "dx", "dw"):
            if hasattr(layer, name) and getattr(layer, name) is not None:
                self.register_buffer(name, getattr(layer, name).detach().cpu().float().clone())
        self.geom = (layer.kernel_size, layer.stride, layer.padding, layer.dilation)
        self.grad = layer.grad
        self.m = layer.scale_momentum
        self.update_scale = layer.update_scale
        self.weight_bits = layer.weight_bits

    def forward(self, x):
        B = x.shape[0]
        k, s, p, d = self.geom
        O = self.weight.shape[0]
        tx = getattr(self, "dx", None)
        tw = getattr(self, "dw", None)
        if self.qtype == "int8":
            qmax_w = 2 ** (self.weight_bits - 1) - 1
            if self.training and self.update_scale:
                with torch.no_grad():
                    cur = x.abs().max() / 127.0
                    self.scale_x.copy_(self.m * cur + (1 - self.m) * self.scale_x)
                    am = self.weight.abs().amax(dim=(1, 2, 3))
                    cw = torch.where(am > 0, am / qmax_w, self.scale_w)
                    self.scale_w.copy_(self.m * cw + (1 - self.m) * self.scale_w)
            qx = _FQ.apply(x, self.scale_x, -127, 127, None)
            qw = _FQ.apply(self.weight, self.scale_w.view(-1, 1, 1, 1), -qmax_w, qmax_w, None)
            y = _LUTConv.apply(qx, qw, self.lut, self.geom, 128, 0.0, self.grad, tx, tw)
        else:
            qmax_w = 2 ** self.weight_bits - 1
            qx = _FQ.apply(x, self.scale_x, 0, 255, self.zero_x)
            qw = _FQ.apply(self.weight, self.scale_w.view(-1, 1, 1, 1), 0, qmax_w,
                           self.zero_w.view(-1, 1, 1, 1))
            y = _LUTConv.apply(qx, qw, self.lut, self.geom, 0, float(self.zero_x), self.grad,
                               tx, tw)
            xp = F.pad(qx - self.zero_x, (p[1], p[1], p[0], p[0])) + self.zero_x
            xsum = F.unfold(xp, k, dilation=d, stride=s).sum(dim=1)
            wu = qw.reshape(O, -1)
            zw = self.zero_w.view(1, -1, 1)
            y = y - zw * xsum.unsqueeze(1) - (self.zero_x * wu.sum(1)).view(1, -1, 1) \
                + wu.shape[1] * self.zero_x * zw
        OH = (x.shape[2] + 2 * p[0] - d[0] * (k[0] - 1) - 1) // s[0] + 1
        OW = (x.shape[3] + 2 * p[1] - d[1] * (k[1] - 1) - 1) // s[1] + 1
        y = y.view(B, O, OH, OW) * (self.scale_x * self.scale_w).view(1, -1, 1, 1)
        return y if self.bias is None else y + self.bias.view(1, -1, 1, 1)


def to_cpu_reference(model):
    """Deep-copies a converted model to the CPU with every approximate conv
    replaced by its torch-CPU twin."""
    import copy
    from approxtorch_amd.nn import Conv2d_int8, Conv2d_uint8
    swaps = {n: LUTConv2dCPU(m) for n, m in model.named_modules()
             if isinstance(m, (Conv2d_int8, Conv2d_uint8))}
    saved = {}
    for n in swaps:
        parent, attr = (n.rsplit(".", 1) if "." in n else ("", n))
        pm = model.get_submodule(parent) if parent else model
        saved[n] = getattr(pm, attr)
        setattr(pm, attr, nn.Identity())
    cpu = copy.deepcopy(model).cpu()
    for n, m in saved.items():
        parent, attr = (n.rsplit(".", 1) if "." in n else ("", n))
        setattr(model.get_submodule(parent) if parent else model, attr, m)
        setattr(cpu.get_submodule(parent) if parent else cpu, attr, swaps[n])
    return cpu
