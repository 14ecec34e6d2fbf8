"""Text LUT loaders (approxtorch/load_lut.py:5-55).

A multiplier LUT file holds 256 rows of 256 integers, row = activation
value (+128 for int8), column = weight value.  Gradient tables are float32
text files (256 values for LRE, 256 x 256 for custom gradients).  The files
are parsed by the library's native parser (atx_parse_text_table): the same
numbers numpy.loadtxt reads, ValueError on a malformed file or a wrong count.
"""
from typing import Literal

import numpy as np
import torch

from .backend import ops


def _read(path, integral, shape=None):
    vals = ops.parse_text_table(path, integral=integral)
    if shape is not None:
        n = int(np.prod(shape))
        if vals.size != n:
            raise ValueError(f"{path}: expected {n} values, found {vals.size}")
        vals = vals.reshape(shape)
    return vals


def load_lut(file_path, qtype: Literal['int8', 'int4', 'uint8'] = 'int8'):
    shape = 256 if qtype in ('int8', 'uint8') else 16
    lut_array = _read(file_path, True, (shape, shape)).astype(np.int32)
    lut_tensor = torch.tensor(lut_array).view(shape * shape).to(torch.int)
    lut_tensor.requires_grad_(False)
    return lut_tensor


def load_lre_grad_lut(da_file_path, db_file_path):
    da = torch.tensor(_read(da_file_path, False)).view(-1)
    db = torch.tensor(_read(db_file_path, False)).view(-1)
    da.requires_grad_(False)
    db.requires_grad_(False)
    return da, db


def load_half_custom_grad_lut(file_path):
    return torch.tensor(_read(file_path, False)).view(-1)


def load_custom_grad_lut(dx_file_path, dw_file_path):
    """Pair-wise custom gradients indexed [x + 128, w + 128] (int8) or [x, w]."""
    dx = torch.tensor(_read(dx_file_path, False)).view(-1)
    dw = torch.tensor(_read(dw_file_path, False)).view(-1)
    dx.requires_grad_(False)
    dw.requires_grad_(False)
    return dx, dw
