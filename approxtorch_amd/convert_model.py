"""Replace nn.Conv2d layers with approximate convolutions (the API of
approxtorch/convert_model.py:15-221).

The conversion is two-phase: every selected conv is turned into its
replacement first, and only when all of them were built are they installed
in their parents, so a conv the layers cannot express (string padding, a
non-zero padding mode, an unsupported group count) raises and leaves the
model as it was.  A replacement adopts its source's parameters (cloned, with
their requires_grad), its device (for every buffer except the caller's
tables), its weight quantization parameters (re-derived from the adopted
weight) and its train/eval flag.

Extension: qtype="uint8" accepts weight_bits 1..8 (the reference fixes 8).
"""
from typing import Literal

import torch
import torch.nn as nn

from .nn import Conv2d_int8, Conv2d_uint8

QType = Literal["int8", "uint8"]
GradType = Literal["ste", "lre", "custom"]

_LAYER = {"int8": Conv2d_int8, "uint8": Conv2d_uint8}


def _validate(model, lut, qtype, grad, ignore_first_conv, update_scale, scale_momentum,
              weight_bits):
    """Argument checks, all before the model is looked at."""
    if not isinstance(model, nn.Module):
        raise TypeError(f"model must be an nn.Module, got {type(model).__name__}")
    if not isinstance(lut, torch.Tensor):
        raise TypeError(f"lut must be a torch.Tensor, got {type(lut).__name__}")
    if lut.numel() != 256 * 256:
        raise ValueError(f"lut must have 65536 elements, got {lut.numel()}")
    if qtype not in _LAYER:
        raise ValueError(f"qtype must be 'int8' or 'uint8', got {qtype!r}")
    if grad not in ("ste", "lre", "custom"):
        raise ValueError(f"grad must be 'ste', 'lre' or 'custom', got {grad!r}")
    for flag, value in (("ignore_first_conv", ignore_first_conv),
                        ("update_scale", update_scale)):
        if not isinstance(value, bool):
            raise TypeError(f"{flag} must be a bool")
    if not 0.0 <= scale_momentum <= 1.0:
        raise ValueError(f"scale_momentum must be between 0 and 1, got {scale_momentum}")
    if isinstance(weight_bits, bool) or not isinstance(weight_bits, int):
        raise TypeError("weight_bits must be an int")
    if qtype == "int8" and not 3 <= weight_bits <= 8:
        raise ValueError(f"weight_bits must be between 3 and 8, got {weight_bits}")
    if qtype == "uint8" and not 1 <= weight_bits <= 8:
        raise ValueError(f"weight_bits must be between 1 and 8 for uint8, got {weight_bits}")


def _conv_sites(root):
    """(parent, attribute, conv) of every nn.Conv2d under root, in the order
    of root.named_modules() and each module once (a module reachable by
    several paths is found at the first); parent is None for the root."""
    visited = set()

    def walk(parent, attr, module):
        if id(module) in visited:
            return
        visited.add(id(module))
        if isinstance(module, nn.Conv2d):
            yield parent, attr, module
        for name, child in module._modules.items():
            if child is not None:
                yield from walk(module, name, child)

    yield from walk(None, None, root)


def _adopted(param):
    return nn.Parameter(param.detach().clone(memory_format=torch.preserve_format),
                        requires_grad=param.requires_grad)


def _replacement(source, layer_cls, lut, options):
    """A layer_cls computing what `source` computes, on source's device."""
    if isinstance(source.padding, str):
        raise NotImplementedError(
            f"convert_model does not support Conv2d string padding {source.padding!r}")
    if source.padding_mode != "zeros":
        raise NotImplementedError(
            f"convert_model only supports Conv2d padding_mode='zeros', got {source.padding_mode!r}")
    layer = layer_cls(source.in_channels, source.out_channels, source.kernel_size, lut,
                      bias=source.bias is not None, stride=source.stride,
                      padding=source.padding, dilation=source.dilation, groups=source.groups,
                      **options)
    device = source.weight.device
    for name, buf in list(layer._buffers.items()):
        if buf is not None and name not in layer.caller_tables:
            layer._buffers[name] = buf.to(device=device)
    layer.weight = _adopted(source.weight)
    if source.bias is not None:
        layer.bias = _adopted(source.bias)
    layer.reset_weight_qparams()
    layer.train(source.training)
    return layer


def convert_model(model: nn.Module, lut: torch.Tensor, qtype: QType = "int8",
                  grad: GradType = "ste", dx: torch.Tensor | None = None,
                  dw: torch.Tensor | None = None, ignore_first_conv: bool = True,
                  scale_momentum: float = 0.05, update_scale: bool = True,
                  weight_bits: int = 8) -> nn.Module:
    """Replace selected nn.Conv2d layers with Conv2d_int8 / Conv2d_uint8.

    int8: per-tensor symmetric activations, per-channel symmetric weights;
    uint8: per-tensor asymmetric activations, per-channel asymmetric weights.
    The model is modified in place and returned (a bare nn.Conv2d model
    returns its replacement).  Convert before building the optimizer: the
    replacements own new Parameter objects."""
    _validate(model, lut, qtype, grad, ignore_first_conv, update_scale, scale_momentum,
              weight_bits)
    sites = list(_conv_sites(model))
    if ignore_first_conv:
        sites = sites[1:]
    options = dict(grad=grad, dx=dx, dw=dw, update_scale=update_scale,
                   scale_momentum=scale_momentum, weight_bits=weight_bits)
    built = [(parent, attr, _replacement(conv, _LAYER[qtype], lut, options))
             for parent, attr, conv in sites]
    result = model
    for parent, attr, layer in built:
        if parent is None:
            result = layer
        else:
            setattr(parent, attr, layer)
    return result
