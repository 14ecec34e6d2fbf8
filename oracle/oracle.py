"""CPU oracle of the LUT approximate-multiplier path — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline);
the product path (approxtorch_amd) never imports it.

Each function restates one piece of the reference's algorithm (citations
relative to approxtorch/ of woshimark666/ApproxTorch) in numpy, or calls the
C restatement in lut_oracle.c for the int64 LUT sums.  Integer quantities are
computed exactly (int64); floating-point quantities follow the reference's
fp32 operation order where bit-exactness is meaningful (fake-quant, EMA,
qparams) and fp64 elsewhere (gradients, used with a tolerance).

Pinning (tests/test_oracle.py): every function here is checked against a
closed form, a brute-force evaluation, an invariant or a hand-computed
special case; none is "parity unpinned".
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")
_lib = None


def _c():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} missing: run `make -C oracle`")
        _lib = ctypes.CDLL(_LIB_PATH)
        vp, ci = ctypes.c_void_p, ctypes.c_int
        _lib.oracle_lut_gemm_i64.argtypes = [vp, vp, vp, ci, ci, ci, ci, vp]
        _lib.oracle_lut_gemm_f32.argtypes = [vp, vp, vp, ci, ci, ci, ci, vp]
        _lib.oracle_custom_grads_f64.argtypes = [vp, vp, vp, vp, vp, ci, ci, ci, ci, vp, vp]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ LUT sums
def lut_gemm_i64(xi, wi, lut):
    """y[n,o,l] = sum_k lut[xi[n,k,l]*256 + wi[o,k]] in exact int64.
    csrc/naive_cuda/bgemm_naive.cu:32-58; NAIVE-README:15-56 (lut[x][w])."""
    xi = np.ascontiguousarray(xi, dtype=np.uint8)
    wi = np.ascontiguousarray(wi, dtype=np.uint8)
    lut = np.ascontiguousarray(np.asarray(lut).reshape(-1), dtype=np.int64)
    N, K, L = xi.shape
    O = wi.shape[0]
    y = np.empty((N, O, L), dtype=np.int64)
    if y.size:
        _c().oracle_lut_gemm_i64(_p(xi), _p(wi), _p(lut), N, K, L, O, _p(y))
    return y


def lut_gemm_f32(xi, wi, lut):
    """fp32 sum in ascending k, the reference's non-split order
    (csrc/claude/bgemm_lut_kernels.cuh:276-284)."""
    xi = np.ascontiguousarray(xi, dtype=np.uint8)
    wi = np.ascontiguousarray(wi, dtype=np.uint8)
    lut = np.ascontiguousarray(np.asarray(lut).reshape(-1), dtype=np.float32)
    N, K, L = xi.shape
    O = wi.shape[0]
    y = np.empty((N, O, L), dtype=np.float32)
    if y.size:
        _c().oracle_lut_gemm_f32(_p(xi), _p(wi), _p(lut), N, K, L, O, _p(y))
    return y


def lut_gemm_bruteforce(xi, wi, lut):
    """Pure-Python triple loop (tiny inputs only) — the oracle of the oracle."""
    lut = np.asarray(lut).reshape(-1)
    N, K, L = xi.shape
    O = wi.shape[0]
    y = np.zeros((N, O, L), dtype=object)
    for n in range(N):
        for o in range(O):
            for l in range(L):
                s = 0
                for k in range(K):
                    s += int(lut[int(xi[n, k, l]) * 256 + int(wi[o, k])])
                y[n, o, l] = s
    return y


def lut_class(lut):
    """0 = int16, 1 = uint16, 2 = fp32 fallback (csrc/claude/bgemm_lut_kernels.cuh:116-142)."""
    v = np.asarray(lut, dtype=np.float32).reshape(-1)
    is_int = v == np.rint(v)
    if np.all(is_int & (np.abs(v) <= 32767)):
        return 0
    if np.all(is_int & (v >= 0) & (v <= 65535)):
        return 1
    return 2


# ------------------------------------------------------------- index images
def quant_index(v, offset):
    """clamp(rint(v) + offset, 0, 255) (csrc/claude/bgemm_lut_kernels.cuh:62-67)."""
    r = np.rint(np.asarray(v, dtype=np.float32))
    r = np.where(np.isnan(r), 0, r)
    return np.clip(np.clip(r, -1024, 1024).astype(np.int64) + offset, 0, 255).astype(np.uint8)


def image_index(img, offset=128):
    """Index image of a quantized image: int8 -> v+128, uint8 -> v,
    fp32 -> quant_index(v, offset) (csrc/claude/bgemm_lre_backward_claude.cu:64-78)."""
    img = np.asarray(img)
    if img.dtype == np.int8:
        return (img.astype(np.int64) + 128).astype(np.uint8)
    if img.dtype == np.uint8:
        return img.copy()
    return quant_index(img, offset)


def out_size(H, W, k, s, p, d):
    OH = (H + 2 * p[0] - d[0] * (k[0] - 1) - 1) // s[0] + 1
    OW = (W + 2 * p[1] - d[1] * (k[1] - 1) - 1) // s[1] + 1
    return OH, OW


def im2col_index(idx_img, k, s, p, d, pad_index=128):
    """[N,C,H,W] index image -> [N, C*kh*kw, OH*OW], k order (c, kh, kw),
    out-of-image taps = pad_index (csrc/claude/bgemm_lre_backward_claude.cu:215-269)."""
    N, C, H, W = idx_img.shape
    OH, OW = out_size(H, W, k, s, p, d)
    padded = np.full((N, C, H + 2 * p[0], W + 2 * p[1]), pad_index, dtype=idx_img.dtype)
    padded[:, :, p[0]:p[0] + H, p[1]:p[1] + W] = idx_img
    cols = np.empty((N, C, k[0], k[1], OH, OW), dtype=idx_img.dtype)
    for i in range(k[0]):
        for j in range(k[1]):
            hs, ws = i * d[0], j * d[1]
            cols[:, :, i, j] = padded[:, :, hs:hs + s[0] * (OH - 1) + 1:s[0],
                                      ws:ws + s[1] * (OW - 1) + 1:s[1]]
    return cols.reshape(N, C * k[0] * k[1], OH * OW)


def unfold_values(img, k, s, p, d, pad_value=0.0):
    """fp64 unfold of a value image with a constant border (F.unfold after padding)."""
    N, C, H, W = img.shape
    OH, OW = out_size(H, W, k, s, p, d)
    padded = np.full((N, C, H + 2 * p[0], W + 2 * p[1]), pad_value, dtype=np.float64)
    padded[:, :, p[0]:p[0] + H, p[1]:p[1] + W] = img
    cols = np.empty((N, C, k[0], k[1], OH, OW), dtype=np.float64)
    for i in range(k[0]):
        for j in range(k[1]):
            hs, ws = i * d[0], j * d[1]
            cols[:, :, i, j] = padded[:, :, hs:hs + s[0] * (OH - 1) + 1:s[0],
                                      ws:ws + s[1] * (OW - 1) + 1:s[1]]
    return cols.reshape(N, C * k[0] * k[1], OH * OW)


def fold(col, shape, k, s, p, d):
    """F.fold: scatter-add of col [N, C*kh*kw, L] into an image [N,C,H,W] (fp64)."""
    N, C, H, W = shape
    OH, OW = out_size(H, W, k, s, p, d)
    padded = np.zeros((N, C, H + 2 * p[0], W + 2 * p[1]), dtype=np.float64)
    c6 = np.asarray(col, dtype=np.float64).reshape(N, C, k[0], k[1], OH, OW)
    for i in range(k[0]):
        for j in range(k[1]):
            hs, ws = i * d[0], j * d[1]
            padded[:, :, hs:hs + s[0] * (OH - 1) + 1:s[0],
                   ws:ws + s[1] * (OW - 1) + 1:s[1]] += c6[:, :, i, j]
    return padded[:, :, p[0]:p[0] + H, p[1]:p[1] + W]


def lut_map(idx, table):
    """out = table[idx] (csrc/claude/bgemm_lre_backward_claude.cu:95-127)."""
    return np.asarray(table, dtype=np.float32)[np.asarray(idx, dtype=np.int64)]


def lut_map_pad(idx_img, table, p):
    """Mapped image with constant border table[128]
    (csrc/claude/bgemm_lre_backward_claude.cu:276-307)."""
    table = np.asarray(table, dtype=np.float32)
    N, C, H, W = idx_img.shape
    out = np.full((N, C, H + 2 * p[0], W + 2 * p[1]), table[128], dtype=np.float32)
    out[:, :, p[0]:p[0] + H, p[1]:p[1] + W] = table[idx_img.astype(np.int64)]
    return out


# ---------------------------------------------------------------- fake-quant
f32 = np.float32


def fakequant(x, scale, qmin, qmax, zero=None):
    """(q, mask): v = x / max(s, 1e-12) (+ z); q = clamp(rint(v)); mask on v.
    nn/quantization.py:37-91; csrc/claude/quantization.cu:54-75."""
    x = np.asarray(x, dtype=f32)
    s = np.maximum(np.asarray(scale, dtype=f32), f32(1e-12))
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        v = (x / s).astype(f32)
        if zero is not None:
            v = (v + np.asarray(zero, dtype=f32)).astype(f32)
        mask = (v >= qmin) & (v <= qmax)
        q = np.clip(np.rint(v), f32(qmin), f32(qmax)).astype(f32)
    return q, mask


def fakequant_backward(go, mask, scale):
    """gx = (mask ? go : 0) / max(s, 1e-12) (csrc/claude/quantization.cu:112-143)."""
    s = np.maximum(np.asarray(scale, dtype=f32), f32(1e-12))
    return (np.where(mask, np.asarray(go, dtype=f32), f32(0)) / s).astype(f32)


# ------------------------------------------------ fp16 / bf16 activations
def round_to(v, dtype):
    """fp32 values rounded to dtype ("f16" or "bf16", round to nearest even;
    bf16 NaN -> the canonical 0x7fc0) and returned as fp32: the value torch
    stores for an elementwise result of that dtype computed in fp32."""
    v = np.asarray(v, dtype=f32)
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return v.astype(np.float16).astype(f32)
    if dtype == "bf16":
        u = v.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
        r = np.where(np.isnan(v), np.uint32(0x7FC00000), r).astype(np.uint32)
        return r.view(f32)
    raise ValueError(dtype)


def fakequant_lowp(x, scale, qmin, qmax, dtype, zero=None):
    """(q, mask) of an fp16 / bf16 x with 0-dim scale (and zero point): the
    reference's unfused statements (nn/quantization.py:44-52,72-80) as torch
    evaluates them in that dtype -- s = clamp(scale, 1e-12) cast to it, v =
    x / s rounded to it (+ zero cast to it, rounded), mask on v, q =
    clamp(round(v)).  x holds the dtype's values as fp32."""
    x = np.asarray(x, dtype=f32)
    s = round_to(np.maximum(f32(scale), f32(1e-12)), dtype)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        v = round_to(x / s, dtype)
        if zero is not None:
            v = round_to(v + round_to(f32(zero), dtype), dtype)
        mask = (v >= qmin) & (v <= qmax)
        q = np.clip(np.rint(v), f32(qmin), f32(qmax)).astype(f32)
    return q, mask


def fakequant_lowp_backward(go, mask, scale, dtype):
    """grad_x = grad_output * mask.to(dtype) / s in dtype (nn/quantization.py:
    58-62): go (fp32 or the dtype's values) rounded to the dtype as autograd
    casts it, the exact product with the mask, the quotient by s cast to the
    dtype rounded to it."""
    g = round_to(go, dtype)
    s = round_to(np.maximum(f32(scale), f32(1e-12)), dtype)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        gm = (g * np.asarray(mask, dtype=f32)).astype(f32)
        return round_to(gm / s, dtype)


def ema_absmax_lowp(x, scale_x, m, dtype, denom=127.0):
    """nn/Conv2d_int8.py:137-146 for an x of dtype: abs_max is a scalar of
    that dtype, so cur = abs_max / denom and m * cur are rounded to it;
    (1 - m) * scale_x and the sum are fp32 (the 0-dim tensors promote)."""
    x = np.asarray(x, dtype=f32)
    absmax = np.max(np.abs(x)) if not np.isnan(x).any() else f32(np.nan)
    cur = round_to(div_by_number(absmax, denom), dtype)
    a = round_to(f32(m) * cur, dtype)
    b = f32(f32(1 - m) * f32(scale_x))
    return f32(f32(a) + b)


def weight_scale_ema_lowp(w, scale_w, m, qmax_w, dtype, reset=False):
    """nn/Conv2d_int8.py:148-158 (reset: 160-167) for an fp16 / bf16 weight:
    absmax / qmax_w is rounded to the weight's dtype, torch.where with the fp32
    scale promotes it back exactly, the EMA is fp32."""
    w = np.asarray(w, dtype=f32).reshape(w.shape[0], -1)
    absmax = np.abs(w).max(axis=1)
    cur_d = round_to(div_by_number(absmax, qmax_w), dtype)
    if reset:
        return np.where(absmax > 0, cur_d, f32(1)).astype(f32)
    cur = np.where(absmax > 0, cur_d, scale_w).astype(f32)
    a = (f32(m) * cur).astype(f32)
    b = (f32(1 - m) * np.asarray(scale_w, dtype=f32)).astype(f32)
    return (a + b).astype(f32)


def ema_scalar(m, cur, old):
    """m*cur + (1-m)*old with both python scalars cast to fp32 and each
    operation rounded to fp32 (the torch op sequence of nn/Conv2d_int8.py:145)."""
    a = f32(f32(m) * f32(cur))
    b = f32(f32(1 - m) * f32(old))
    return f32(a + b)


def div_by_number(v, number):
    """`tensor / number` (number a python scalar) as torch evaluates it on the
    GPU: v * fp32(1 / fp32(number)), rounded to fp32 (its true-divide kernel
    multiplies by the reciprocal when the divisor is a host scalar; exact
    division differs in the last bit for a few percent of values)."""
    return (np.asarray(v, dtype=f32) * (f32(1) / f32(number))).astype(f32)


def ema_absmax(x, scale_x, m, denom=127.0):
    """nn/Conv2d_int8.py:137-146, the statements as torch runs them on the
    GPU (abs_max / 127 through div_by_number)."""
    x = np.asarray(x, dtype=f32)
    absmax = np.max(np.abs(x)) if not np.isnan(x).any() else f32(np.nan)
    cur = f32(div_by_number(absmax, denom))
    return ema_scalar(m, cur, scale_x)


def weight_scale_ema(w, scale_w, m, qmax_w):
    """nn/Conv2d_int8.py:148-158 (zero channels keep their scale)."""
    w = np.asarray(w, dtype=f32).reshape(w.shape[0], -1)
    absmax = np.abs(w).max(axis=1)
    cur = np.where(absmax > 0, div_by_number(absmax, qmax_w), scale_w).astype(f32)
    a = (f32(m) * cur).astype(f32)
    b = (f32(1 - m) * np.asarray(scale_w, dtype=f32)).astype(f32)
    return (a + b).astype(f32)


def weight_scale_reset(w, qmax_w):
    """nn/Conv2d_int8.py:160-167."""
    w = np.asarray(w, dtype=f32).reshape(w.shape[0], -1)
    absmax = np.abs(w).max(axis=1)
    return np.where(absmax > 0, div_by_number(absmax, qmax_w), f32(1)).astype(f32)


def uint8_qparams(mn, mx, qmax=255):
    """nn/Conv2d_uint8.py:11-23."""
    mn = np.minimum(np.asarray(mn, dtype=f32), f32(0))
    mx = np.maximum(np.asarray(mx, dtype=f32), f32(0))
    scale = np.maximum(div_by_number((mx - mn).astype(f32), qmax), f32(1e-12)).astype(f32)
    zero = np.clip(np.rint((-mn / scale).astype(f32)), f32(0), f32(qmax)).astype(f32)
    return scale, zero


def ema_minmax(x, x_min, x_max, m, qmax=255):
    """nn/Conv2d_uint8.py:225-240 -> (x_min', x_max', scale, zero)."""
    x = np.asarray(x, dtype=f32)
    nmin = ema_scalar(m, x.min(), x_min)
    nmax = ema_scalar(m, x.max(), x_max)
    s, z = uint8_qparams(nmin, nmax, qmax)
    return nmin, nmax, s, z


def weight_minmax_ema(w, w_min, w_max, m, qmax=255):
    """nn/Conv2d_uint8.py:242-255."""
    w2 = np.asarray(w, dtype=f32).reshape(w.shape[0], -1)
    a = (f32(m) * w2.min(axis=1)).astype(f32) + (f32(1 - m) * w_min).astype(f32)
    b = (f32(m) * w2.max(axis=1)).astype(f32) + (f32(1 - m) * w_max).astype(f32)
    a, b = a.astype(f32), b.astype(f32)
    s, z = uint8_qparams(a, b, qmax)
    return a, b, s, z


# ----------------------------------------------------------- GEMM gradients
def gemm_grads(go, xi, wi, kind, tables=None, signed=True, absolute=False):
    """fp64 gradients of y = sum_k f(xi, wi) for the three estimators.
    STE: nn/bgemm_int8.py:15-25 (values idx-128, or idx for uint8);
    LRE: csrc/naive_cuda/bgeem_lre_navie.cu:28-88 / NAIVE-README:222-232
         (grad_x uses dx[wi], grad_w uses dw[xi]);
    custom: csrc/naive_cuda/bgemm_custom_grad_naive.cu:28-92
         (dx_lut[xi][wi], dw_lut[xi][wi]; evaluated by lut_oracle.c).
    absolute=True evaluates the same sums over |go| and |tables| (the sum of
    |terms| of each output, which bounds any fp32 summation order's error).
    Returns grad_x [N,K,L], grad_w [O,K]."""
    go = np.asarray(go, dtype=np.float64)
    if absolute:
        go = np.abs(go)
    xi = np.ascontiguousarray(xi, dtype=np.uint8)
    wi = np.ascontiguousarray(wi, dtype=np.uint8)
    if kind in ("ste", "lre"):
        if kind == "ste":
            off = 128 if signed else 0
            tx = np.arange(256, dtype=np.float64) - off
            tw = tx
        else:
            tx = np.asarray(tables[0], dtype=np.float64).reshape(-1)
            tw = np.asarray(tables[1], dtype=np.float64).reshape(-1)
        if absolute:
            tx, tw = np.abs(tx), np.abs(tw)
        a = tx[wi.astype(np.int64)]                          # [O, K]
        gx = np.matmul(a.T[None], go)                        # [N, K, L]
        b = tw[xi.astype(np.int64)]                          # [N, K, L]
        gw = np.matmul(go, b.transpose(0, 2, 1)).sum(axis=0)  # [O, K]
        return gx, gw
    dxl = np.ascontiguousarray(np.asarray(tables[0], dtype=np.float64).reshape(-1))
    dwl = np.ascontiguousarray(np.asarray(tables[1], dtype=np.float64).reshape(-1))
    if absolute:
        dxl, dwl = np.abs(dxl), np.abs(dwl)
    go = np.ascontiguousarray(go)
    N, K, L = xi.shape
    O = wi.shape[0]
    gx = np.zeros((N, K, L), dtype=np.float64)
    gw = np.zeros((O, K), dtype=np.float64)
    if gx.size and gw.size:
        _c().oracle_custom_grads_f64(_p(xi), _p(wi), _p(go), _p(dxl), _p(dwl), N, K, L, O,
                                     _p(gx), _p(gw))
    return gx, gw


# ---------------------------------------------------------------- the layers
def conv_int8_forward(x, weight, bias, lut, scale_x, scale_w, k, s, p, d, weight_bits=8,
                      x_dtype=None):
    """Conv2d_int8.forward with given scales (nn/Conv2d_int8.py:171-220).
    Returns y (fp64), and the intermediates needed by the backward.  x_dtype
    "f16" / "bf16": x holds that dtype's values and is fake-quantized in it
    (fakequant_lowp); the weight stays fp32 (its per-channel scale promotes)."""
    qmax_w = 2 ** (weight_bits - 1) - 1
    if x_dtype is None:
        qx, mx = fakequant(x, scale_x, -127, 127)
    else:
        qx, mx = fakequant_lowp(x, scale_x, -127, 127, x_dtype)
    O = weight.shape[0]
    qw, mw = fakequant(weight, np.asarray(scale_w, dtype=f32).reshape(O, 1, 1, 1), -qmax_w,
                       qmax_w)
    xi = im2col_index(image_index(qx, 128), k, s, p, d, 128)
    wi = image_index(qw.reshape(O, -1), 128)
    acc = lut_gemm_i64(xi, wi, lut)                          # [N, O, L] exact
    sc = (f32(scale_x) * np.asarray(scale_w, dtype=f32)).astype(f32)
    N, _, H, W = x.shape
    OH, OW = out_size(H, W, k, s, p, d)
    y = acc.astype(np.float64) * sc.astype(np.float64)[None, :, None]
    yabs = np.abs(y)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :, None]
        yabs = yabs + np.abs(np.asarray(bias, dtype=np.float64))[None, :, None]
    # yabs: sum of |terms| of each output (tolerance bound of fp32 evaluations)
    ctx = dict(xi=xi, wi=wi, mx=mx, mw=mw, sc=sc, shape=x.shape, acc=acc,
               yabs=yabs.reshape(N, O, OH, OW))
    return y.reshape(N, O, OH, OW), ctx


def conv_int8_backward(go, ctx, scale_x, scale_w, kind, tables, k, s, p, d, absolute=False,
                       x_dtype=None):
    """Gradients of the int8 layer (fp64): the reference's composition of the
    fake-quant STE backward, the conv Function backward (nn/bgemm_int8.py
    conv level) and the dequant addcmul.  absolute=True gives the sum of
    |terms| of every gradient element instead (a tolerance bound).  x_dtype
    "f16" / "bf16": gx is the x fake-quant's gradient in that dtype
    (fakequant_lowp_backward of the fp32-rounded gradient of the quantized x;
    with absolute, the bound of that gradient before the STE, divided by s)."""
    N, O = go.shape[:2]
    go = np.abs(go) if absolute else go
    g = np.asarray(go, dtype=np.float64).reshape(N, O, -1) * \
        ctx["sc"].astype(np.float64)[None, :, None]
    gcol, gwq = gemm_grads(g, ctx["xi"], ctx["wi"], kind, tables, signed=True,
                           absolute=absolute)
    gqx = fold(gcol, ctx["shape"], k, s, p, d)
    sx = max(float(f32(scale_x)), 1e-12)
    if x_dtype is not None and not absolute:
        gx = fakequant_lowp_backward(gqx.astype(f32), ctx["mx"], scale_x, x_dtype)
    else:
        gx = np.where(ctx["mx"], gqx, 0.0) / sx
    sw = np.maximum(np.asarray(scale_w, dtype=np.float64), 1e-12)
    gw = np.where(ctx["mw"].reshape(O, -1), gwq, 0.0) / sw[:, None]
    gb = np.asarray(go, dtype=np.float64).sum(axis=(0, 2, 3))
    return gx, gw.reshape(ctx["mw"].shape), gb


def dwconv_int8_forward(x, weight, bias, lut, scale_x, scale_w, k, s, p, d, weight_bits=8):
    """Depthwise Conv2d_int8 (groups == C == O): the LUT conv run per channel,
    which is how the reference defines its depthwise kernel
    (csrc/claude/dwconv_claude.cu:3-12; nn/Conv2d_int8.py:35-41,198-205)."""
    C = x.shape[1]
    bias = None if bias is None else np.asarray(bias)
    sw = np.asarray(scale_w, dtype=f32).reshape(-1)
    ys, ctxs = [], []
    for c in range(C):
        y, ctx = conv_int8_forward(x[:, c:c + 1], weight[c:c + 1],
                                   None if bias is None else bias[c:c + 1], lut, scale_x,
                                   sw[c:c + 1], k, s, p, d, weight_bits)
        ys.append(y)
        ctxs.append(ctx)
    return np.concatenate(ys, axis=1), ctxs


def dwconv_yabs(ctxs):
    """Sum of |terms| of each depthwise output (tolerance bound)."""
    return np.concatenate([c["yabs"] for c in ctxs], axis=1)


def dwconv_int8_backward(go, ctxs, scale_x, scale_w, kind, tables, k, s, p, d,
                         absolute=False):
    """Gradients of the depthwise layer: conv_int8_backward per channel."""
    sw = np.asarray(scale_w, dtype=f32).reshape(-1)
    parts = [conv_int8_backward(go[:, c:c + 1], ctxs[c], scale_x, sw[c:c + 1], kind, tables,
                                k, s, p, d, absolute) for c in range(len(ctxs))]
    return (np.concatenate([q[0] for q in parts], axis=1),
            np.concatenate([q[1] for q in parts], axis=0),
            np.concatenate([q[2] for q in parts], axis=0))


def conv_uint8_forward(x, weight, bias, lut, scale_x, zero_x, scale_w, zero_w, k, s, p, d,
                       qmax_w=255):
    """Conv2d_uint8.forward with given qparams (nn/Conv2d_uint8.py:257-325)."""
    qx, mx = fakequant(x, scale_x, 0, 255, zero=zero_x)
    O = weight.shape[0]
    qw, mw = fakequant(weight, np.asarray(scale_w, dtype=f32).reshape(O, 1, 1, 1), 0, qmax_w,
                       zero=np.asarray(zero_w, dtype=f32).reshape(O, 1, 1, 1))
    zx = int(np.rint(zero_x))
    xi = im2col_index(image_index(qx, 0), k, s, p, d, zx)
    wi = image_index(qw.reshape(O, -1), 0)
    lutsum = lut_gemm_i64(xi, wi, lut).astype(np.float64)
    K = wi.shape[1]
    xsum = xi.astype(np.float64).sum(axis=1)                 # [N, L]
    wsum = wi.astype(np.float64).sum(axis=1)                 # [O]
    zw = np.asarray(zero_w, dtype=np.float64)
    zxf = float(zero_x)
    terms = (lutsum, zw[None, :, None] * xsum[:, None, :], (zxf * wsum)[None, :, None],
             K * zxf * zw[None, :, None])
    y = terms[0] - terms[1] - terms[2] + terms[3]
    yabs = sum(np.abs(v) for v in terms)
    sc = (f32(scale_x) * np.asarray(scale_w, dtype=f32)).astype(f32)
    y = y * sc.astype(np.float64)[None, :, None]
    yabs = yabs * sc.astype(np.float64)[None, :, None]
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :, None]
        yabs = yabs + np.abs(np.asarray(bias, dtype=np.float64))[None, :, None]
    N, _, H, W = x.shape
    OH, OW = out_size(H, W, k, s, p, d)
    # yabs: sum of |terms| of each output (tolerance bound of fp32 evaluations)
    ctx = dict(xi=xi, wi=wi, mx=mx, mw=mw, sc=sc, shape=x.shape, zw=zw, zx=zxf,
               yabs=np.broadcast_to(yabs, (N, O, yabs.shape[2])).reshape(N, O, OH, OW))
    return y.reshape(N, O, OH, OW), ctx


def conv_uint8_backward(go, ctx, scale_x, scale_w, kind, tables, k, s, p, d, absolute=False):
    """Gradients of the uint8 layer (fp64) including the zero-point terms that
    autograd adds through xsum / wsum (nn/Conv2d_uint8.py:36-51,308-315).
    absolute=True gives the sum of |terms| of every gradient element."""
    N, O = go.shape[:2]
    go = np.abs(go) if absolute else go
    g = np.asarray(go, dtype=np.float64).reshape(N, O, -1) * \
        ctx["sc"].astype(np.float64)[None, :, None]
    gcol, gwq = gemm_grads(g, ctx["xi"], ctx["wi"], kind, tables, signed=False,
                           absolute=absolute)
    sign = 1.0 if absolute else -1.0
    # -z_w * xsum  ->  d xu[n,k,l] -= sum_o z_w[o] g[n,o,l]
    gcol = gcol + sign * np.einsum("o,nol->nl", ctx["zw"], g)[:, None, :]
    # -z_x * wsum  ->  d wu[o,k] -= z_x * sum_{n,l} g[n,o,l]
    gwq = gwq + sign * ctx["zx"] * g.sum(axis=(0, 2))[:, None]
    gqx = fold(gcol, ctx["shape"], k, s, p, d)
    sx = max(float(f32(scale_x)), 1e-12)
    gx = np.where(ctx["mx"], gqx, 0.0) / sx
    sw = np.maximum(np.asarray(scale_w, dtype=np.float64), 1e-12)
    gw = np.where(ctx["mw"].reshape(O, -1), gwq, 0.0) / sw[:, None]
    gb = np.asarray(go, dtype=np.float64).sum(axis=(0, 2, 3))
    return gx, gw.reshape(ctx["mw"].shape), gb


# ------------------------------------------------------------ gradient tables
def lre_tables(lut, qtype="int8"):
    """OLS slopes per LUT column (grad_a) and row (grad_b) (grad_lut.py:14-37)."""
    lut = np.asarray(lut, dtype=np.float32).reshape(256, 256).astype(np.float64)
    vals = np.arange(-128, 128, dtype=np.float64) if qtype == "int8" else \
        np.arange(256, dtype=np.float64)
    xc = vals - vals.mean()
    den = (xc * xc).sum()
    grad_a = (xc[:, None] * (lut - lut.mean(axis=0, keepdims=True))).sum(axis=0) / den
    grad_b = (xc[None, :] * (lut - lut.mean(axis=1, keepdims=True))).sum(axis=1) / den
    return grad_a.astype(np.float32), grad_b.astype(np.float32)


def date_tables(lut, half_ws):
    """grad_lut.py:39-142 restated with explicit loops (float32 storage)."""
    lut = np.asarray(lut, dtype=np.float32).reshape(256, 256)

    def smooth(line):
        out = line.copy()
        for i in range(256):
            if half_ws <= i <= 255 - half_ws:
                out[i] = line[i - half_ws:i + half_ws + 1].mean(dtype=np.float32)
        return out

    def diff(line):
        out = np.empty(256, dtype=np.float32)
        fb = f32((line[-1] - line[0]) / f32(255.0))
        for i in range(256):
            out[i] = (line[i + 1] - line[i - 1]) / f32(2.0) if half_ws < i < 255 - half_ws \
                else fb
        return out

    ga = np.empty((256, 256), dtype=np.float32)
    gb = np.empty((256, 256), dtype=np.float32)
    for b in range(256):
        ga[:, b] = diff(smooth(lut[:, b]))
    for a in range(256):
        gb[a, :] = diff(smooth(lut[a, :]))
    return ga, gb
