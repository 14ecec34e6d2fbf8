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

`multiplier` may be a text-file path (as in the reference) or a 256 x 256
array / tensor.  Extension: lre also handles qtype='uint8' (operands 0..255);
the reference returns None there.
"""
import numpy as np


def _as_table(multiplier):
    if isinstance(multiplier, np.ndarray):
        lut = multiplier
    elif hasattr(multiplier, "detach"):
        lut = multiplier.detach().cpu().numpy()
    else:
        lut = np.loadtxt(multiplier, dtype=np.float32)
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
    lut = _as_table(multiplier)
    grad_a = _diff(_smooth(lut.T.copy(), half_ws), half_ws).T.copy()
    grad_b = _diff(_smooth(lut.copy(), half_ws), half_ws)
    if save_path is not None:
        np.savetxt(f'{save_path}_date_{half_ws}_grad_a.txt', grad_a)
        np.savetxt(f'{save_path}_date_{half_ws}_grad_b.txt', grad_b)
    return grad_a.astype(np.float32), grad_b.astype(np.float32)
