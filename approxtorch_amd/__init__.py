"""approxtorch_amd: LUT approximate-multiplier convolutions for AMD Instinct
MI355X (gfx950).

Public API of approxtorch kept intact: convert_model, nn.Conv2d_int8 /
nn.Conv2d_uint8, load_lut, grad_lut, the autograd Functions in
nn.bgemm_int8 / nn.bgemm_uint8 / nn.quantization and backend.ops.  All
compute runs in libatx.so (hand-written HIP for gfx950).
"""
from . import backend
from . import nn
from .convert_model import convert_model
from . import load_lut
from . import grad_lut
from . import calib

__all__ = ["backend", "nn", "convert_model", "load_lut", "grad_lut", "calib"]
