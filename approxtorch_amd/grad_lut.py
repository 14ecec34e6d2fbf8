"""Gradient-table generators for the LRE and custom (DATE) estimators.

lre(multiplier, qtype, save_path)   approxtorch/grad_lut.py:14-37
    grad_a[y] = least-squares slope of LUT[:, y] over the row operand
    (used as dx, indexed by the weight), grad_b[x] = slope of LUT[x, :]
    over the column operand (used as dw, indexed by the activation).
    The slope is the closed-form OLS estimate sum((x-xm)(y-ym)) / sum((x-xm)^2),
    the quantity scipy.stats.linregress returns as `slope`.
DATE(multiplier, half_ws, save_path)   approxtorch/grad_lut.py:39-142
    (2h+1)-tap moving average along one axis (identity within h of the
    edges), then central differences inside (h, 255-h) and the end-to-end
    slope (s[255]-s[0])/255 elsewhere.

`multiplier` may be a text-file path (as in the reference), a 256 x 256
array, or a tensor.  A CUDA tensor is handled on the device by the
library's generators (ops.lre_tables / ops.date_tables, cached per LUT) and
gives CUDA tensors; the other inputs give numpy arrays as in the reference,
the same values (the device DATE kernel reproduces numpy's float32 window
means).  Extension: lre also handles qtype='uint8' (operands 0..255); the
reference returns None there.
"""
import numpy as np
import torch

from .backend import ops


def _device_lut(multiplier):
    if isinstance(multiplier, torch.Tensor) and multiplier.is_cuda:
        return multiplier.detach().to(torch.float32).reshape(-1).contiguous()
    return None


def _as_table(multiplier):
    if isinstance(multiplier, np.ndarray):
        lut = multiplier
    elif hasattr(multiplier, "detach"):
        lut = multiplier.detach().cpu().numpy()
    else:
        lut = ops.parse_text_table(multiplier)
    lut = np.asarray(lut, dtype=np.float32).reshape(256, 256)
    return lut


def _ols_slopes(values, lines):
    """Slope of each row of `lines` (shape [m, 256]) against `values` ([256])."""
    x = values.astype(np.float64)
    y = lines.astype(np.float64)
    xm = x.mean()
    ym = y.mean(axis=1, keepdims=True)
    return ((x - xm) * (y - ym)).sum(axis=1) / ((x - xm) ** 2).sum()


def lre(multiplier, qtype, save_path=None):
    dev = _device_lut(multiplier)
    if dev is not None and qtype in ('int8', 'uint8'):
        grad_a, grad_b = ops.lre_tables(dev, qtype)
        if save_path is not None:
            np.savetxt(f'{save_path}_lre_grad_a.txt', grad_a.cpu().numpy(), fmt='%.4f')
            np.savetxt(f'{save_path}_lre_grad_b.txt', grad_b.cpu().numpy(), fmt='%.4f')
        return grad_a.clone(), grad_b.clone()
    lut = _as_table(multiplier)
    if qtype == 'int8':
        vals = np.arange(-128, 128)
    elif qtype == 'uint8':
        vals = np.arange(0, 256)
    else:
        return None
    grad_a = _ols_slopes(vals, lut.T).astype(np.float32)   # column y: LUT[:, y]
    grad_b = _ols_slopes(vals, lut).astype(np.float32)     # row x: LUT[x, :]
    if save_path is not None:
        np.savetxt(f'{save_path}_lre_grad_a.txt', grad_a, fmt='%.4f')
        np.savetxt(f'{save_path}_lre_grad_b.txt', grad_b, fmt='%.4f')
    return grad_a, grad_b


def _smooth(lines, half_ws):
    """Moving average of each row (float32, numpy's own mean per window)."""
    out = lines.copy()
    w = 2 * half_ws + 1
    if w <= 256:
        win = np.lib.stride_tricks.sliding_window_view(lines, w, axis=1)
        out[:, half_ws:256 - half_ws] = win.mean(axis=-1, dtype=np.float32)
    return out


def _diff(smooth_lines, half_ws):
    grad = np.empty_like(smooth_lines)
    fallback = (smooth_lines[:, -1] - smooth_lines[:, 0]) / np.float32(255.0)
    grad[:] = fallback[:, None]
    lo, hi = half_ws + 1, 255 - half_ws        # central difference for lo <= i < hi
    if hi > lo:
        grad[:, lo:hi] = (smooth_lines[:, lo + 1:hi + 1] - smooth_lines[:, lo - 1:hi - 1]) \
            / np.float32(2.0)
    return grad


def DATE(multiplier, half_ws=32, save_path=None):
    """Smoothing + difference gradients: returns (grad_a, grad_b), each 256 x 256
    float32, the derivative along the row operand a and the column operand b."""
    dev = _device_lut(multiplier)
    if dev is not None and 0 <= half_ws <= 127:
        ga, gb = ops.date_tables(dev, half_ws)
        ga, gb = ga.view(256, 256).clone(), gb.view(256, 256).clone()
        if save_path is not None:
            np.savetxt(f'{save_path}_date_{half_ws}_grad_a.txt', ga.cpu().numpy())
            np.savetxt(f'{save_path}_date_{half_ws}_grad_b.txt', gb.cpu().numpy())
        return ga, gb
    lut = _as_table(multiplier)
    grad_a = _diff(_smooth(lut.T.copy(), half_ws), half_ws).T.copy()
    grad_b = _diff(_smooth(lut.copy(), half_ws), half_ws)
    if save_path is not None:
        np.savetxt(f'{save_path}_date_{half_ws}_grad_a.txt', grad_a)
        np.savetxt(f'{save_path}_date_{half_ws}_grad_b.txt', grad_b)
    return grad_a.astype(np.float32), grad_b.astype(np.float32)
