"""Tensor-level wrappers over the C ABI, named after the reference's ops.

Each wrapper mirrors one op of approxtorch/backend/ops.py (and the schema it
binds in csrc/), checks arguments the way the reference's TORCH_CHECKs do
(RuntimeError), allocates outputs with torch on the input's device and
launches the HIP kernels on the current stream.  The GEMM operands are
re-laid out for the gfx950 kernels (row-offset activations, transposed
weights) inside these wrappers; callers see the reference's shapes.
"""
import os
import threading
import weakref

import torch
from torch import Tensor
from torch.nn.modules.utils import _pair

from . import _lib as L

__all__ = [
    "lut_image", "bgemm_fake_int8_claude", "bgemm_fake_int8_claude_save",
    "bgemm_fake_uint8_claude", "bgemm_fake_uint8_claude_save", "bgemm_fake_int8_claude_cfg",
    "bgemm_fake_uint8_claude_cfg", "lut_gemm_i32", "im2col_u8", "lut_map", "lut_map_pad",
    "bgemm_lre_backward_claude", "bgemm_lre_backward_claude_cfg",
    "bgemm_lre_backward_claude_im2col", "bgemm_custom_grad_uint8_dx", "bgemm_custom_grad_uint8_dw",
    "bgemm_custom_grad_int8_dx", "bgemm_custom_grad_int8_dw", "custom_grads", "pack_rows_u8", "fakequant_per_tensor",
    "fakequant_per_tensor_backward", "fakequant_per_channel", "conv_forward",
    "conv_backward_data", "conv_backward_weight", "conv_backward_weight_rows", "col2im",
    "gemm_fake_int8_claude",
    "gemm_fake_int8_claude_save", "gemm_fake_int8_claude_cfg", "gemm_fake_uint8_claude",
    "gemm_fake_uint8_claude_save", "gemm_fake_uint8_claude_cfg", "dwconv_fake_int8_claude",
    "dwconv_forward", "dwconv_backward_data", "dwconv_backward_weight", "parse_text_table",
    "lre_tables", "date_tables",
]

# --------------------------------------------------------------------- LUTs
# Derived device tables (the 16-bit LUT image, LRE / DATE tables) are cached
# per LUT tensor.  An entry is keyed by everything that determines the bytes a
# kernel would read -- storage address, offset, shape, strides, version --
# and holds only a weak reference to the LUT's storage, so it goes stale (and
# is recomputed) when that memory is freed and its address reused.  The cache is
# unbounded: a converted ResNet-50 holds one LUT copy per layer after
# Module.to(), and a bounded LRU smaller than that would miss on every call.
# Edits that bypass the version counter (through .data) are not seen.
_LUT_CACHE = {}
_LUT_LOCK = threading.Lock()


def _check_lut(lut, name="lut"):
    if not lut.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if lut.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32")
    if lut.numel() != 256 * 256:
        raise RuntimeError(f"{name} must have 65536 elements")


def _cache_key(kind, lut, param):
    return (kind, param, lut.data_ptr(), lut.device.index, lut.storage_offset(),
            tuple(lut.shape), tuple(lut.stride()), lut._version)


def _cached(kind, lut, param, make):
    """make(lut.contiguous()) cached per (LUT tensor, kind, param)."""
    _check_lut(lut)
    key = _cache_key(kind, lut, param)
    storage = lut.untyped_storage()
    with _LUT_LOCK:
        hit = _LUT_CACHE.get(key)
        if hit is not None and hit[0]() is storage:
            return hit[1]
    val = make(lut.contiguous())
    with _LUT_LOCK:
        for k in [k for k, v in _LUT_CACHE.items() if v[0]() is None]:
            del _LUT_CACHE[k]
        _LUT_CACHE[key] = (weakref.ref(storage), val)
    return val


def lut_image(lut: Tensor, transposed: bool = False):
    """(lut16t, lutf32t, class) for an fp32 [65536] LUT, cached per tensor.

    The 16-bit transposed image and its class (int16 / uint16 / fp32
    fallback) are computed once per LUT tensor -- the reference rebuilds them
    inside every forward (csrc/claude/bgemm_float_claude.cu:161-192).
    transposed=True gives the image of the transposed LUT (lut[w][x] roles
    swapped), for a GEMM whose row operand is the LUT's second index.
    """
    def make(lc):
        if transposed:
            lc = lc.view(256, 256).t().contiguous().view(-1)
        dev = lc.device
        img16 = torch.empty(65536, dtype=torch.int16, device=dev)
        imgf = torch.empty(65536, dtype=torch.float32, device=dev)
        flags = torch.zeros(2, dtype=torch.int32, device=dev)
        L.call("atx_lut_prepare", L.ptr(lc), L.ptr(img16), L.ptr(imgf), L.ptr(flags),
               L.stream_of(lc))
        f = flags.tolist()          # one host sync per new LUT tensor
        cls = L.ATX_LUT_I16 if f[0] == 0 else (L.ATX_LUT_U16 if f[1] == 0 else L.ATX_LUT_F32)
        return img16, imgf, cls
    return _cached("image", lut, bool(transposed), make)


# ------------------------------------------------ LUT files and gradient tables
def parse_text_table(path, integral=False, capacity=1 << 24):
    """fp32 numpy array of the numbers in a text table file (whitespace or
    comma separated, '#' comments): the native replacement of the
    numpy.loadtxt calls in load_lut.py:5-55.  Malformed files raise ValueError
    (numpy.loadtxt's error type)."""
    import numpy as np
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not found.")
    out = np.empty(capacity, dtype=np.float32)
    count = np.zeros(1, dtype=np.int64)
    lib = L.load()
    rc = lib.atx_parse_text_table(os.fsencode(os.fspath(path)), int(bool(integral)),
                                  out.ctypes.data, capacity, count.ctypes.data)
    if rc != 0:
        raise ValueError(lib.atx_last_error().decode(errors="replace"))
    return out[:int(count[0])].copy()


def lre_tables(lut: Tensor, qtype: str = "int8"):
    """(grad_a [256], grad_b [256]) LRE slope tables of a CUDA fp32 LUT, on the
    device, cached per LUT (grad_lut.py:14-37; uint8 operands: qtype='uint8')."""
    if qtype not in ("int8", "uint8"):
        raise ValueError(f"qtype must be 'int8' or 'uint8', got {qtype!r}")
    offset = 128 if qtype == "int8" else 0

    def launch(lc):
        ga = torch.empty(256, dtype=torch.float32, device=lc.device)
        gb = torch.empty(256, dtype=torch.float32, device=lc.device)
        L.call("atx_lre_tables", L.ptr(lc), offset, L.ptr(ga), L.ptr(gb), L.stream_of(lc))
        return ga, gb
    return _cached("lre", lut, offset, launch)


def date_tables(lut: Tensor, half_ws: int = 32):
    """(grad_a, grad_b) [65536] DATE tables of a CUDA fp32 LUT, on the device,
    cached per LUT (grad_lut.py:39-142)."""
    if not 0 <= half_ws <= 127:
        raise ValueError(f"half_ws must be in [0, 127], got {half_ws}")

    def launch(lc):
        ga = torch.empty(65536, dtype=torch.float32, device=lc.device)
        gb = torch.empty(65536, dtype=torch.float32, device=lc.device)
        L.call("atx_date_tables", L.ptr(lc), half_ws, L.ptr(ga), L.ptr(gb), L.stream_of(lc))
        return ga, gb
    return _cached("date", lut, half_ws, launch)


# -------------------------------------------------------------- LUT GEMM
def _gemm(xt, Rpad, wt, Opad, N, K, Lc, O, lut, out_kind, y, sx=None, sw=None, bias=None,
          transposed=False, wbase=None, x_upper=None, u8=None):
    """wbase: the caller guarantees every weight index lies in [wbase, wbase + 16)
    (weight_bits <= 4); integer LUTs then run on the matrix cores.  x_upper: a
    device int32 flag that, when nonzero, guarantees every activation index of
    the rows is >= 128 (atx_gemm_epilogue.x_upper; upper-half tables).
    u8 = (xsum, wsum, zero_x, zero_w): the uint8 layer's zero-point correction
    and dequant by sx * sw (+ bias) into the fp32 y, in the matrix-core GEMM's
    epilogue when it runs (wbase 0, integer LUT), else as atx_uint8_dequant
    after the fp32 sums; the same values either way."""
    img16, imgf, cls = lut_image(lut, transposed)
    dev = y.device
    if u8 is not None:
        xsum, wsum, zx, zw = u8
        if wbase == 0 and cls != L.ATX_LUT_F32 and K > 0:
            wsb = L.query("atx_lut_gemm_narrow_workspace_bytes", N, K, Lc, O)
            ws = torch.empty(max(wsb // 4, 1), dtype=torch.int32, device=dev) if wsb else None
            L.call("atx_lut_gemm_narrow_uint8", L.ptr(xt), Rpad, L.ptr(wt), Opad, N, K, Lc, O,
                   L.ptr(img16), cls, L.ptr(sx), L.ptr(sw), L.ptr(bias), L.ptr(xsum),
                   L.ptr(wsum), L.ptr(zx), L.ptr(zw), L.ptr(y), L.ptr(ws), L.stream_of(y))
            return y
        _gemm(xt, Rpad, wt, Opad, N, K, Lc, O, lut, L.ATX_OUT_F32, y, transposed=transposed,
              wbase=wbase, x_upper=x_upper)
        uint8_dequant(y, xsum, wsum, zx, zw, sx, sw, bias, K)
        return y
    ep = L.GemmEpilogue(out_kind, L.ptr(sx), L.ptr(sw), L.ptr(bias), L.ptr(x_upper))
    if wbase is not None and cls != L.ATX_LUT_F32:
        wsb = L.query("atx_lut_gemm_narrow_workspace_bytes", N, K, Lc, O)
        ws = torch.empty(max(wsb // 4, 1), dtype=torch.int32, device=dev) if wsb else None
        L.call("atx_lut_gemm_narrow", L.ptr(xt), Rpad, L.ptr(wt), Opad, N, K, Lc, O,
               L.ptr(img16), cls, int(wbase), ep, L.ptr(y), L.ptr(ws), L.stream_of(y))
        return y
    wsb = L.query("atx_lut_gemm_workspace_bytes", N, K, Lc, O) if cls != L.ATX_LUT_F32 else 0
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.int32, device=dev) if wsb else None
    L.call("atx_lut_gemm", L.ptr(xt), Rpad, L.ptr(wt), Opad, N, K, Lc, O, L.ptr(img16),
           L.ptr(imgf), cls, ep, L.ptr(y), L.ptr(ws), L.stream_of(y))
    return y


def upper_flag(device):
    """A device int32 flag set to 1, for a fake-quant or row-packing kernel to
    clear when some LUT index of its operand is below 128; passed on as the
    LUT GEMM's x_upper, a flag still set lets it build half-height tables
    (atx_gemm_epilogue.x_upper)."""
    return torch.ones((), dtype=torch.int32, device=device)


def _pack_w(w, offset, want_wq=True, want_wt=True):
    """w fp32 [O,K] (quantized values) or uint8 [O,K] indices -> (wq, wt, Opad);
    want_wt=False (fp32 w) writes wq alone and returns wt None."""
    O, K = w.shape
    Opad = L.round_up(max(O, 1), L.COL_TILE)
    s = L.stream_of(w)
    if not want_wt and w.dtype != torch.uint8:
        wq = torch.empty((O, K), dtype=torch.uint8, device=w.device)
        L.call("atx_pack_w_f32", L.ptr(w), O, K, offset, L.ptr(wq), None, Opad, s)
        return wq, None, Opad
    wt = torch.empty((K, Opad), dtype=torch.uint8, device=w.device)
    if w.dtype == torch.uint8:
        L.call("atx_pack_w_u8", L.ptr(w), O, K, L.ptr(wt), Opad, s)
        return w, wt, Opad
    wq = torch.empty((O, K), dtype=torch.uint8, device=w.device) if want_wq else None
    L.call("atx_pack_w_f32", L.ptr(w), O, K, offset, L.ptr(wq), L.ptr(wt), Opad, s)
    return wq, wt, Opad


def _bgemm_save(x, w, lut, offset, name):
    # checks of csrc/claude/bgemm_float_claude.cu:80-91
    if not (x.is_cuda and w.is_cuda and lut.is_cuda):
        raise RuntimeError(f"{name}: x, w and lut must be CUDA tensors")
    if x.dtype not in (torch.float32, torch.uint8):
        raise RuntimeError("x must be float32 or uint8 (LUT indices)")
    if w.dtype != torch.float32:
        raise RuntimeError("w must be float32")
    _check_lut(lut)
    if x.dim() != 3:
        raise RuntimeError("x must have shape [N, CKK, L]")
    if w.dim() != 2:
        raise RuntimeError("w must have shape [O, CKK]")
    if x.size(1) != w.size(1):
        raise RuntimeError("x.size(1) must equal w.size(1)")
    xc, wc = x.contiguous(), w.contiguous()
    N, K, Lc = xc.shape
    O = wc.size(0)
    dev, s = xc.device, L.stream_of(xc)
    R = N * Lc
    Rpad = L.round_up(max(R, 1), L.ROW_TILE)
    xt = torch.empty((L.operand_rows(K), Rpad), dtype=torch.int16, device=dev)
    up = upper_flag(dev)
    if xc.dtype == torch.uint8:
        xq = xc
        L.call("atx_pack_x_u8", L.ptr(xc), N, K, Lc, L.ptr(xt), Rpad, L.ptr(up), s)
    else:
        xq = torch.empty((N, K, Lc), dtype=torch.uint8, device=dev)
        L.call("atx_pack_x_f32", L.ptr(xc), N, K, Lc, offset, L.ptr(xq), L.ptr(xt), Rpad,
               L.ptr(up), s)
    wq, wt, Opad = _pack_w(wc, offset)
    y = torch.empty((N, O, Lc), dtype=torch.float32, device=dev)
    _gemm(xt, Rpad, wt, Opad, N, K, Lc, O, lut, L.ATX_OUT_F32, y, x_upper=up)
    return y, xq, wq


def bgemm_fake_int8_claude_save(X: Tensor, W: Tensor, lut: Tensor):
    """(y, xq, wq): y[n,o,l] = sum_k lut[(x+128)*256 + (w+128)], plus the uint8
    index images (xq aliases X when X is uint8).  csrc/claude/bgemm_float_claude.cu:209-241."""
    return _bgemm_save(X, W, lut, 128, "bgemm_fake_int8_claude_save")


def bgemm_fake_int8_claude(X: Tensor, W: Tensor, lut: Tensor) -> Tensor:
    return bgemm_fake_int8_claude_save(X, W, lut)[0]


def bgemm_fake_int8_claude_cfg(X: Tensor, W: Tensor, lut: Tensor, cfg: int) -> Tensor:
    """`cfg` selected one of the reference's CUDA tile configurations; the gfx950
    kernel has a single tiling, so it is accepted and ignored."""
    return bgemm_fake_int8_claude(X, W, lut)


def bgemm_fake_uint8_claude_save(X: Tensor, W: Tensor, lut: Tensor):
    """uint8 x uint8 variant: lut[x*256 + w] with raw values as indices.
    csrc/claude/bgemm_float_claude.cu:245-277."""
    return _bgemm_save(X, W, lut, 0, "bgemm_fake_uint8_claude_save")


def bgemm_fake_uint8_claude(X: Tensor, W: Tensor, lut: Tensor) -> Tensor:
    return bgemm_fake_uint8_claude_save(X, W, lut)[0]


def bgemm_fake_uint8_claude_cfg(X: Tensor, W: Tensor, lut: Tensor, cfg: int) -> Tensor:
    return bgemm_fake_uint8_claude(X, W, lut)


def lut_gemm_i32(X: Tensor, W: Tensor, lut: Tensor) -> Tensor:
    """Exact int32 LUT sums for uint8 index operands X [N,K,L], W [O,K]
    (integer LUT classes only)."""
    if X.dtype != torch.uint8 or W.dtype != torch.uint8:
        raise RuntimeError("lut_gemm_i32 takes uint8 index operands")
    xc, wc = X.contiguous(), W.contiguous()
    N, K, Lc = xc.shape
    O = wc.size(0)
    Rpad = L.round_up(max(N * Lc, 1), L.ROW_TILE)
    xt = torch.empty((L.operand_rows(K), Rpad), dtype=torch.int16, device=xc.device)
    up = upper_flag(xc.device)
    L.call("atx_pack_x_u8", L.ptr(xc), N, K, Lc, L.ptr(xt), Rpad, L.ptr(up), L.stream_of(xc))
    _, wt, Opad = _pack_w(wc, 0)
    y = torch.empty((N, O, Lc), dtype=torch.int32, device=xc.device)
    return _gemm(xt, Rpad, wt, Opad, N, K, Lc, O, lut, L.ATX_OUT_I32, y, x_upper=up)


# ------------------------------------------- plain LUT GEMM (torch.mm layout)
def _gemm2d_save(A, B, lut, offset, name):
    """y [M,N] = sum_k lut[idx(A[m,k]) * 256 + idx(B[k,n])] and the u8 images
    aq [M,K] (aliases a contiguous uint8 A) and bq [N,K] (B transposed):
    csrc/claude/gemm.cu:93-230.  A, B: fp32 quantized values or uint8 indices,
    any strides.  The rows of the gfx950 tile (2048 deep) run along the larger
    of M and N: rows = M reads A as the row operand and writes y as N_b = M
    images of one position (y[m][n] = out[m][n][0]); rows = N reads B^T as the
    row operand with the transposed LUT image, and y = out[0][m][n]."""
    if not (A.is_cuda and B.is_cuda and lut.is_cuda):
        raise RuntimeError(f"{name}: A, B and lut must be CUDA tensors")
    for nm, t in (("A", A), ("B", B)):
        if t.dtype not in (torch.float32, torch.uint8):
            raise RuntimeError(f"{nm} must be float32 or uint8 (LUT indices)")
    _check_lut(lut)
    if A.dim() != 2:
        raise RuntimeError("A must have shape [M, K]")
    if B.dim() != 2:
        raise RuntimeError("B must have shape [K, N]")
    if A.size(1) != B.size(0):
        raise RuntimeError(f"A.size(1) must equal B.size(0), got {A.size(1)} vs {B.size(0)}")
    M, K = A.shape
    N = B.size(1)
    if max(M, K, N) > 2 ** 31 - 1:
        raise RuntimeError("dimensions too large")
    dev, s = A.device, L.stream_of(A)
    u8 = dict(dtype=torch.uint8, device=dev)
    a_u8 = A.dtype == torch.uint8
    aq = A.contiguous() if a_u8 else torch.empty((M, K), **u8)
    bq = torch.empty((N, K), **u8)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    rows_m = M >= N
    if rows_m:
        R, C, Nb, Lc = M, N, M, 1
        X, sr, sk, xq = A, A.stride(0), A.stride(1), None if a_u8 else aq
        Y, sc, skc, yq = B, B.stride(1), B.stride(0), bq
    else:
        R, C, Nb, Lc = N, M, 1, N
        X, sr, sk, xq = B, B.stride(1), B.stride(0), bq
        Y, sc, skc, yq = A, A.stride(0), A.stride(1), None if a_u8 else aq
    Rpad = L.round_up(max(R, 1), L.ROW_TILE)
    Opad = L.round_up(max(C, 1), L.COL_TILE)
    xt = torch.empty((L.operand_rows(K), Rpad), dtype=torch.int16, device=dev)
    wt = torch.empty((K, Opad), **u8)
    up = upper_flag(dev)
    L.call("atx_pack_rows_strided", L.ptr(X), int(X.dtype == torch.uint8), R, K, sr, sk,
           offset, L.ptr(xq), L.ptr(xt), Rpad, L.ptr(up), s)
    L.call("atx_pack_cols_strided", L.ptr(Y), int(Y.dtype == torch.uint8), C, K, sc, skc,
           offset, L.ptr(yq), L.ptr(wt), Opad, s)
    if y.numel():
        _gemm(xt, Rpad, wt, Opad, Nb, K, Lc, C, lut, L.ATX_OUT_F32, y, transposed=not rows_m,
              x_upper=up)
    return y, aq, bq


def gemm_fake_int8_claude_save(A: Tensor, B: Tensor, lut: Tensor):
    """(y, aq, bq): y[m,n] = sum_k lut[(A[m,k]+128)*256 + (B[k,n]+128)]
    (csrc/claude/gemm.cu:1-40, 232-262)."""
    return _gemm2d_save(A, B, lut, 128, "gemm_fake_int8_claude_save")


def gemm_fake_int8_claude(A: Tensor, B: Tensor, lut: Tensor) -> Tensor:
    return gemm_fake_int8_claude_save(A, B, lut)[0]


def gemm_fake_int8_claude_cfg(A: Tensor, B: Tensor, lut: Tensor, cfg: int) -> Tensor:
    """`cfg` forced one of the reference's CUDA tile configurations or
    orientations; the gfx950 kernel picks its orientation from the shape, so
    it is accepted and ignored."""
    return gemm_fake_int8_claude(A, B, lut)


def gemm_fake_uint8_claude_save(A: Tensor, B: Tensor, lut: Tensor):
    """uint8 x uint8 variant: y[m,n] = sum_k lut[A[m,k]*256 + B[k,n]]
    (csrc/claude/gemm.cu:264-290)."""
    return _gemm2d_save(A, B, lut, 0, "gemm_fake_uint8_claude_save")


def gemm_fake_uint8_claude(A: Tensor, B: Tensor, lut: Tensor) -> Tensor:
    return gemm_fake_uint8_claude_save(A, B, lut)[0]


def gemm_fake_uint8_claude_cfg(A: Tensor, B: Tensor, lut: Tensor, cfg: int) -> Tensor:
    return gemm_fake_uint8_claude(A, B, lut)


# ------------------------------------------------------------- conv path
_DTYPE_CODE = {torch.int8: 0, torch.uint8: 1, torch.float32: 2}


def _dtype_code(t, unsigned=False):
    """Kernel dtype code; fp32 images hold signed (index v+128) or, with
    unsigned=True, unsigned (index v) quantized values."""
    code = _DTYPE_CODE.get(t.dtype)
    if code is None:
        raise RuntimeError(f"unsupported dtype {t.dtype} (int8, uint8 or float32)")
    return 3 if (code == 2 and unsigned) else code


def conv_geom(x_shape, kernel_size, stride, padding, dilation):
    N, C, H, W = x_shape
    kh, kw = _pair(kernel_size)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    return L.geom(N, C, H, W, kh, kw, sh, sw, ph, pw, dh, dw)


def conv_forward(img: Tensor, w_idx_or_val: Tensor, lut: Tensor, g, offset: int,
                 pad_index: int, out_kind=L.ATX_OUT_F32, sx=None, sw=None, bias=None,
                 pad_dev=None, packed_w=None, return_operand=False, wbase=None,
                 x_upper=None, u8=None):
    """LUT conv via implicit im2col: y [N, O, OH*OW] = sum_k lut[xi][wi].

    img: quantized image [N,C,H,W] (int8 values, uint8 values or fp32 values;
    offset 128 = signed operands, 0 = unsigned); w: [O, C*KH*KW] fp32
    quantized values or uint8 indices.  Out-of-image taps use pad_index, or
    the device scalar pad_dev when given.  packed_w = (wq, wt, Opad) from the
    fused weight fake-quant skips the weight packing.  Returns (y, wq), wq the
    uint8 weight index image; with return_operand, (y, wq, (xt, Rpad)), the
    row-offset operand for conv_backward_weight_rows.  wbase: every weight
    index lies in [wbase, wbase + 16) (weight_bits <= 4; matrix-core GEMM).
    x_upper: device flag as in _gemm (the image's indices and pad_index are
    all >= 128 when it is set).  u8: the uint8 correction and dequant terms as
    in _gemm (y is then the layer's fp32 output)."""
    imgc = img.contiguous()
    N, K = g.N, g.C * g.KH * g.KW
    Lc = g.OH * g.OW
    O = w_idx_or_val.size(0)
    if w_idx_or_val.size(1) != K:
        raise RuntimeError(f"weight has {w_idx_or_val.size(1)} taps, geometry needs {K}")
    dev = imgc.device
    Rpad = L.round_up(max(N * Lc, 1), L.ROW_TILE)
    xt = torch.empty((L.operand_rows(K), Rpad), dtype=torch.int16, device=dev)
    L.call("atx_im2col_rows", L.ptr(imgc), _dtype_code(imgc, offset == 0), g, pad_index,
           L.ptr(pad_dev), L.ptr(xt), Rpad, L.stream_of(imgc))
    if packed_w is None:
        wq, wt, Opad = _pack_w(w_idx_or_val.contiguous(), offset)
    else:
        wq, wt, Opad = packed_w
    ydt = torch.int32 if out_kind == L.ATX_OUT_I32 else torch.float32
    y = torch.empty((N, O, Lc), dtype=ydt, device=dev)
    _gemm(xt, Rpad, wt, Opad, N, K, Lc, O, lut, out_kind, y, sx, sw, bias, wbase=wbase,
          x_upper=x_upper, u8=u8)
    if return_operand:
        return y, wq, (xt, Rpad)
    return y, wq


def conv_backward_data(go: Tensor, wq: Tensor, table: Tensor, g, mask=None, scale=None,
                       go_sx=None, go_sw=None):
    """grad wrt the image: fold(sum_o go' * table[wq]) with go' = go * (sx * sw[o])
    when go_sx/go_sw are given, and the fake-quant STE (mask ? g : 0) / max(scale, 1e-12)
    fused when mask is given."""
    goc = go.contiguous()
    O = wq.size(0)
    img = torch.empty((g.N, g.C, g.H, g.W), dtype=torch.float32, device=goc.device)
    wsb = L.query("atx_conv_bwd_data_workspace_bytes", g, O)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=goc.device) if wsb else None
    L.call("atx_conv_bwd_data", L.ptr(goc), L.ptr(wq.contiguous()), L.ptr(table), g, O,
           L.ptr(go_sx), L.ptr(go_sw), L.ptr(mask), L.ptr(scale), L.ptr(img), L.ptr(ws),
           L.stream_of(goc))
    return img


def conv_backward_weight(go: Tensor, img: Tensor, table: Tensor, g, O: int, pad_index: int,
                         mask_w=None, scale_w=None, pad_dev=None, unsigned=False,
                         go_sx=None, go_sw=None):
    """grad wrt the weights: sum_{n,l} go' * table[xi] with implicit im2col
    (go' as in conv_backward_data), the per-channel fake-quant STE fused when
    mask_w is given."""
    goc, imgc = go.contiguous(), img.contiguous()
    K = g.C * g.KH * g.KW
    P = g.N * g.OH * g.OW
    gw = torch.empty((O, K), dtype=torch.float32, device=goc.device)
    wsb = L.query("atx_conv_bwd_weight_workspace_bytes", O, K, P)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=goc.device)
    L.call("atx_conv_bwd_weight", L.ptr(goc), L.ptr(imgc), _dtype_code(imgc, unsigned), g, O,
           pad_index, L.ptr(pad_dev), L.ptr(table), L.ptr(go_sx), L.ptr(go_sw), L.ptr(mask_w),
           L.ptr(scale_w), L.ptr(gw), L.ptr(ws), L.stream_of(goc))
    return gw


# ---------------------------------------------------------- depthwise conv
def dwconv_forward(img: Tensor, wq: Tensor, lut: Tensor, g, pad_index: int,
                   out_kind=L.ATX_OUT_F32, sx=None, sw=None, bias=None, unsigned=False):
    """Depthwise LUT conv: y [N,C,OH,OW] = sum_taps lut[xi][wq[c,t]] (taps in
    ascending (i, j); out-of-image taps index pad_index), with the LUT GEMM's
    epilogues (sw / bias per channel).  wq: uint8 [C, KH*KW] indices."""
    imgc = img.contiguous()
    img16, imgf, cls = lut_image(lut)
    ydt = torch.int32 if out_kind == L.ATX_OUT_I32 else torch.float32
    y = torch.empty((g.N, g.C, g.OH, g.OW), dtype=ydt, device=imgc.device)
    ep = L.GemmEpilogue(out_kind, L.ptr(sx), L.ptr(sw), L.ptr(bias))
    L.call("atx_dwconv_fwd", L.ptr(imgc), _dtype_code(imgc, unsigned), g, pad_index,
           L.ptr(wq.contiguous()), L.ptr(img16), L.ptr(imgf), cls, ep, L.ptr(y),
           L.stream_of(imgc))
    return y


def dwconv_fake_int8_claude(x: Tensor, w: Tensor, lut: Tensor, kernel_size, stride=1,
                            padding=0, dilation=1):
    """(y [N,C,OH,OW] fp32, wq [C, kh*kw] uint8): depthwise (groups == C, channel
    multiplier 1) LUT conv of a quantized image (int8 / uint8 / fp32 values)
    with fp32 quantized weights; equal to the LUT-BGEMM run per channel with
    the same tap order (csrc/claude/dwconv_claude.cu:1-285, ops.py:252-263)."""
    if not (x.is_cuda and w.is_cuda and lut.is_cuda):
        raise RuntimeError("x, w and lut must be CUDA tensors")
    if x.dtype not in (torch.float32, torch.int8, torch.uint8):
        raise RuntimeError("x must be float32, int8 or uint8")
    if w.dtype != torch.float32:
        raise RuntimeError("w must be float32")
    _check_lut(lut)
    if x.dim() != 4:
        raise RuntimeError("x must have shape [N, C, H, W]")
    g = conv_geom(tuple(x.shape), kernel_size, stride, padding, dilation)
    if w.dim() != 2 or w.size(0) != g.C or w.size(1) != g.KH * g.KW:
        raise RuntimeError(f"w must have shape [C, kh*kw] = [{g.C}, {g.KH * g.KW}]")
    if g.OH <= 0 or g.OW <= 0:
        raise RuntimeError("empty output geometry")
    wq, _, _ = _pack_w(w.contiguous(), 128, want_wt=False)
    return dwconv_forward(x, wq, lut, g, 128), wq


def dwconv_backward_data(go: Tensor, wq: Tensor, table: Tensor, g, mask=None, scale=None,
                         go_sx=None, go_sw=None) -> Tensor:
    """grad wrt the image of the depthwise conv (go' and the fused STE as in
    conv_backward_data)."""
    goc = go.contiguous()
    gx = torch.empty((g.N, g.C, g.H, g.W), dtype=torch.float32, device=goc.device)
    L.call("atx_dwconv_bwd_data", L.ptr(goc), L.ptr(wq.contiguous()), L.ptr(table), g,
           L.ptr(go_sx), L.ptr(go_sw), L.ptr(mask), L.ptr(scale), L.ptr(gx), L.stream_of(goc))
    return gx


def dwconv_backward_weight(go: Tensor, img: Tensor, table: Tensor, g, pad_index: int,
                           mask_w=None, scale_w=None, pad_dev=None, unsigned=False,
                           go_sx=None, go_sw=None) -> Tensor:
    """grad wrt the depthwise weights [C, KH*KW] (go' and the fused per-channel
    STE as in conv_backward_weight)."""
    goc, imgc = go.contiguous(), img.contiguous()
    gw = torch.empty((g.C, g.KH * g.KW), dtype=torch.float32, device=goc.device)
    wsb = L.query("atx_dwconv_bwd_weight_workspace_bytes", g)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=goc.device)
    L.call("atx_dwconv_bwd_weight", L.ptr(goc), L.ptr(imgc), _dtype_code(imgc, unsigned), g,
           pad_index, L.ptr(pad_dev), L.ptr(table), L.ptr(go_sx), L.ptr(go_sw), L.ptr(mask_w),
           L.ptr(scale_w), L.ptr(gw), L.ptr(ws), L.stream_of(goc))
    return gw


def conv_backward_weight_rows(go: Tensor, operand, table: Tensor, g, O: int, mask_w=None,
                              scale_w=None, go_sx=None, go_sw=None):
    """conv_backward_weight with the activation indices read from the
    forward's row-offset operand `operand` = (xt, Rpad) of conv_forward."""
    xt, Rpad = operand
    goc = go.contiguous()
    K = g.C * g.KH * g.KW
    Lc = g.OH * g.OW
    gw = torch.empty((O, K), dtype=torch.float32, device=goc.device)
    wsb = L.query("atx_conv_bwd_weight_workspace_bytes", O, K, g.N * Lc)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=goc.device)
    L.call("atx_conv_bwd_weight_rows", L.ptr(goc), L.ptr(xt), Rpad, g.N, K, Lc, O, L.ptr(table),
           L.ptr(go_sx), L.ptr(go_sw), L.ptr(mask_w), L.ptr(scale_w), L.ptr(gw), L.ptr(ws),
           L.stream_of(goc))
    return gw


def tap_sum(img: Tensor, g, pad_dev=None) -> Tensor:
    """[N, L] column sums of the unfolded image (uint8 values or fp32 holding
    quantized integers; padding = pad_dev)."""
    ic = img.contiguous()
    if ic.dtype not in (torch.uint8, torch.float32):
        raise RuntimeError(f"tap_sum: image must be uint8 or float32, got {ic.dtype}")
    out = torch.empty((g.N, g.OH * g.OW), dtype=torch.float32, device=ic.device)
    wsb = L.query("atx_tap_sum_workspace_bytes", g)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=ic.device)
    L.call("atx_tap_sum", L.ptr(ic), 1 if ic.dtype == torch.uint8 else 2, g, L.ptr(pad_dev),
           L.ptr(out), L.ptr(ws), L.stream_of(ic))
    return out


def uint8_dequant(y: Tensor, xsum: Tensor, wsum: Tensor, zero_x: Tensor, zero_w: Tensor,
                  scale_x: Tensor, scale_w: Tensor, bias, K: int) -> Tensor:
    """In place on y [N, O, L] (raw LUT sums of a uint8 conv): the zero-point
    correction and dequant of nn/Conv2d_uint8.py:308-325 in one pass."""
    N, O, Lc = y.shape
    tensors = [y, xsum, wsum, zero_x, zero_w, scale_x, scale_w]
    if not all(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() for t in tensors):
        raise RuntimeError("uint8_dequant: all operands must be contiguous CUDA float32")
    L.call("atx_uint8_dequant", L.ptr(y), N, O, Lc, L.ptr(xsum), L.ptr(wsum), L.ptr(zero_x),
           L.ptr(zero_w), L.ptr(scale_x), L.ptr(scale_w), L.ptr(bias), K, L.stream_of(y))
    return y


def zero_point_pos(go: Tensor, scale_x: Tensor, scale_w: Tensor, zero_w: Tensor) -> Tensor:
    """pos [N, L] = sum_o -(scale_x * scale_w[o]) * zero_w[o] * go[n, o, l] for
    go [N, O, L]: the uint8 layer's zero-point position term in backward."""
    goc = go.contiguous()
    N, O, Lc = goc.shape
    pos = torch.empty((N, Lc), dtype=torch.float32, device=goc.device)
    L.call("atx_zero_point_pos", L.ptr(goc), N, O, Lc, L.ptr(scale_x.contiguous()),
           L.ptr(scale_w.contiguous()), L.ptr(zero_w.contiguous()), L.ptr(pos),
           L.stream_of(goc))
    return pos


# channel sums of go in atx_zero_point_terms: at most this many channels
ZERO_POINT_SUM_MAX_O = 8192


def zero_point_terms(go: Tensor, scale_x: Tensor, scale_w: Tensor, zero_w: Tensor,
                     want_pos: bool = True):
    """(pos [N, L] or None, gsum [O]) from one pass over go [N, O, L]: pos as
    zero_point_pos (when want_pos) and gsum[o] = sum_{n,l} go[n, o, l], the
    gradient of the uint8 layer's -z_x * sum_k q_w[o, k] term and of its
    bias, summed in a fixed order."""
    goc = go.contiguous()
    N, O, Lc = goc.shape
    if O > ZERO_POINT_SUM_MAX_O:
        raise RuntimeError(f"zero_point_terms: at most {ZERO_POINT_SUM_MAX_O} channels")
    pos = torch.empty((N, Lc), dtype=torch.float32, device=goc.device) if want_pos else None
    gsum = torch.empty(O, dtype=torch.float32, device=goc.device)
    wsb = L.query("atx_zero_point_terms_workspace_bytes", N, O, Lc)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=goc.device)
    L.call("atx_zero_point_terms", L.ptr(goc), N, O, Lc, L.ptr(scale_x.contiguous()),
           L.ptr(scale_w.contiguous()), L.ptr(zero_w.contiguous()), L.ptr(pos), L.ptr(gsum),
           L.ptr(ws), L.stream_of(goc))
    return pos, gsum


def tap_sum_backward(go: Tensor, g) -> Tensor:
    goc = go.contiguous()
    img = torch.empty((g.N, g.C, g.H, g.W), dtype=torch.float32, device=goc.device)
    L.call("atx_tap_sum_bwd", L.ptr(goc), g, L.ptr(img), L.stream_of(goc))
    return img


def col2im(col: Tensor, g, pos=None, mask=None, scale=None) -> Tensor:
    """F.fold of col [N, C*KH*KW, L]; pos [N, L] (optional) adds its value at
    every tap of a position (tap_sum's backward) and mask / scale fuse the
    per-tensor fake-quant STE (mask ? v : 0) / max(scale, 1e-12)."""
    colc = col.contiguous()
    img = torch.empty((g.N, g.C, g.H, g.W), dtype=torch.float32, device=colc.device)
    if pos is not None:
        pos = pos.contiguous()
        if pos.dtype != torch.float32 or pos.numel() != g.N * g.OH * g.OW:
            raise RuntimeError("col2im: pos must be float32 [N, OH*OW]")
    if mask is not None and (mask.dtype != torch.bool or mask.numel() != img.numel()):
        raise RuntimeError("col2im: mask must be bool of the image's shape")
    L.call("atx_col2im_pos", L.ptr(colc), g, L.ptr(pos), L.ptr(mask), L.ptr(scale), L.ptr(img),
           L.stream_of(colc))
    return img


# ------------------------------------------------------------ index maps
def im2col_u8(feature: Tensor, kernel_size, stride=1, padding=0, dilation=1) -> Tensor:
    """[N,C,H,W] int8/uint8/fp32 -> uint8 LUT indices [N, C*kh*kw, L], padding -> 128.
    csrc/claude/bgemm_lre_backward_claude.cu:737-791."""
    if not feature.is_cuda:
        raise RuntimeError("im2col_u8: feature must be a CUDA tensor")
    if feature.dim() != 4:
        raise RuntimeError("im2col_u8: feature must be [N, C, H, W]")
    fc = feature.contiguous()
    g = conv_geom(fc.shape, kernel_size, stride, padding, dilation)
    if g.OH <= 0 or g.OW <= 0:
        raise RuntimeError("im2col_u8: empty output")
    out = torch.empty((g.N, g.C * g.KH * g.KW, g.OH * g.OW), dtype=torch.uint8,
                      device=fc.device)
    L.call("atx_im2col_u8", L.ptr(fc), _dtype_code(fc), g, L.ptr(out), L.stream_of(fc))
    return out


def lut_map(x: Tensor, lut: Tensor) -> Tensor:
    """out[i] = lut[idx(x[i])] for a [256] table (int8: v+128, uint8: v,
    fp32: clamp(rint(v))+128).  csrc/claude/bgemm_lre_backward_claude.cu:793-807."""
    if not (x.is_cuda and lut.is_cuda):
        raise RuntimeError("lut_map: tensors must be CUDA tensors")
    if lut.dtype != torch.float32 or lut.numel() != 256:
        raise RuntimeError("lut_map: lut must be float32 with 256 elements")
    xc = x.contiguous()
    out = torch.empty(xc.shape, dtype=torch.float32, device=xc.device)
    L.call("atx_lut_map", L.ptr(xc), _dtype_code(xc), xc.numel(), L.ptr(lut.contiguous()),
           L.ptr(out), L.stream_of(xc))
    return out


def lut_map_pad(x: Tensor, lut: Tensor, padding) -> Tensor:
    """lut_map of an image [N,C,H,W] with a constant border lut[128].
    csrc/claude/bgemm_lre_backward_claude.cu:809-848."""
    ph, pw = _pair(padding)
    if x.dim() != 4:
        raise RuntimeError("lut_map_pad: x must be [N, C, H, W]")
    if lut.dtype != torch.float32 or lut.numel() != 256:
        raise RuntimeError("lut_map_pad: lut must be float32 with 256 elements")
    xc = x.contiguous()
    N, C, H, W = xc.shape
    out = torch.empty((N, C, H + 2 * ph, W + 2 * pw), dtype=torch.float32, device=xc.device)
    L.call("atx_lut_map_pad", L.ptr(xc), _dtype_code(xc), N, C, H, W, ph, pw,
           L.ptr(lut.contiguous()), L.ptr(out), L.stream_of(xc))
    return out


# ------------------------------------------------------------ LRE backward
def _weight_index(w: Tensor) -> Tensor:
    """Any reference weight operand (uint8 index, int8 value, fp32 value) ->
    uint8 index image of the same shape."""
    if w.dtype == torch.uint8:
        return w.contiguous()
    if w.dtype == torch.int8:
        return (w.to(torch.int16) + 128).to(torch.uint8).contiguous()
    if w.dtype == torch.float32:
        O, K = w.shape
        wq, _, _ = _pack_w(w.contiguous(), 128, want_wt=False)
        return wq
    raise RuntimeError(f"unsupported weight dtype {w.dtype}")


def _lre_checks(grad_output, x, w, dx, dw, x_dims):
    """csrc/claude/bgemm_lre_backward_claude.cu:547-560 / 664-677."""
    for t, nm in ((grad_output, "grad_output"), (x, "x"), (w, "w"), (dx, "dx"), (dw, "dw")):
        if not t.is_cuda:
            raise RuntimeError("all tensors must be CUDA")
    if not (grad_output.dtype == dx.dtype == dw.dtype == torch.float32):
        raise RuntimeError("grad_output/dx/dw must be float32")
    for t, nm in ((x, "x"), (w, "w")):
        if t.dtype not in (torch.float32, torch.int8, torch.uint8):
            raise RuntimeError(f"{nm} must be float32, int8 or uint8")
    if grad_output.dim() != 3:
        raise RuntimeError("grad_output must have shape [N, O, L]")
    if x.dim() != x_dims:
        raise RuntimeError("x must have shape " + ("[N, K, L]" if x_dims == 3 else "[N, C, H, W]"))
    if w.dim() != 2:
        raise RuntimeError("w must have shape [K, O]")
    if dx.numel() != 256:
        raise RuntimeError("dx must have 256 elements")
    if dw.numel() != 256:
        raise RuntimeError("dw must have 256 elements")


def _lre_grads(go, x_img, w, dx, dw, g, N, K, Lc, O):
    """(grad_x [N,K,L] unfolded, grad_w [K,O]) of the LRE estimator:
    grad_x[n,k,l] = sum_o go[n,o,l] * dx[idx(w[k,o])] and
    grad_w[k,o] = sum_{n,l} go[n,o,l] * dw[idx(x[n,k,l])], out-of-image taps
    of the implicit im2col taking dw[128] (the quantized zero)."""
    dev = go.device
    if N == 0 or K == 0 or Lc == 0 or O == 0:
        return (torch.zeros((N, K, Lc), dtype=torch.float32, device=dev),
                torch.zeros((K, O), dtype=torch.float32, device=dev))
    wq = _weight_index(w.t().contiguous())                 # [O, K] LUT indices
    goc = go.contiguous()
    col = torch.empty((N, K, Lc), dtype=torch.float32, device=dev)
    L.call("atx_conv_bwd_data_col", L.ptr(goc), L.ptr(wq), L.ptr(dx.contiguous()), N, O, K, Lc,
           L.ptr(col), L.stream_of(goc))
    gw = conv_backward_weight(goc, x_img, dw.contiguous(), g, O, 128)
    return col, gw.t().contiguous()


def bgemm_lre_backward_claude(grad_output: Tensor, x: Tensor, w: Tensor, dx: Tensor,
                              dw: Tensor):
    """LRE backward of the LUT BGEMM (csrc/claude/bgemm_lre_backward_claude.cu:539-647):
      grad_x[n,k,l] = sum_o go[n,o,l] * dx[idx(w[k,o])]
      grad_w[k,o]   = sum_{n,l} go[n,o,l] * dw[idx(x[n,k,l])]
    x [N,K,L] and w [K,O] are uint8 indices, int8 values or fp32 values."""
    _lre_checks(grad_output, x, w, dx, dw, 3)
    N, K, Lc = x.shape
    O = w.size(1)
    if w.size(0) != K:
        raise RuntimeError("w.shape[0] must equal K")
    if tuple(grad_output.shape) != (N, O, Lc):
        raise RuntimeError("grad_output shape must be [N, O, L]")
    g = L.geom(N, K, 1, Lc, 1, 1, 1, 1, 0, 0, 1, 1)
    return _lre_grads(grad_output, x.contiguous().view(N, K, 1, Lc), w, dx, dw, g, N, K, Lc, O)


def bgemm_lre_backward_claude_cfg(grad_output: Tensor, x: Tensor, w: Tensor, dx: Tensor,
                                  dw: Tensor, cfg: int):
    """`cfg` chose between the reference's cuBLAS grad_w formulations
    (csrc/claude/bgemm_lre_backward_claude.cu:545,603-611); the gfx950 MFMA
    weight-gradient GEMM picks its own split, so it is accepted and ignored."""
    return bgemm_lre_backward_claude(grad_output, x, w, dx, dw)


def bgemm_lre_backward_claude_im2col(grad_output: Tensor, x: Tensor, w: Tensor, dx: Tensor,
                                     dw: Tensor, kernel_size, stride, padding, dilation):
    """bgemm_lre_backward_claude with x the pre-unfold quantized image
    [N,C,H,W] (int8 / uint8 / fp32 values): the weight-gradient GEMM reads its
    im2col indices on the fly, padding taps = index 128
    (csrc/claude/bgemm_lre_backward_claude.cu:649-733; ops.py:266-275).
    Returns (grad_x [N, C*kh*kw, L] unfolded, grad_w [C*kh*kw, O])."""
    _lre_checks(grad_output, x, w, dx, dw, 4)
    kh, kw = _pair(kernel_size)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw_ = _pair(dilation)
    if not (kh >= 1 and kw >= 1 and sh >= 1 and sw >= 1 and ph >= 0 and pw >= 0 and dh >= 1
            and dw_ >= 1):
        raise RuntimeError("invalid conv geometry")
    xc = x.contiguous()
    g = conv_geom(tuple(xc.shape), (kh, kw), (sh, sw), (ph, pw), (dh, dw_))
    N, K = g.N, g.C * kh * kw
    O = w.size(1)
    if w.size(0) != K:
        raise RuntimeError("w.shape[0] must equal C*kh*kw")
    if g.OH < 1 or g.OW < 1:
        raise RuntimeError("conv geometry yields empty output")
    Lc = g.OH * g.OW
    if tuple(grad_output.shape) != (N, O, Lc):
        raise RuntimeError(f"grad_output shape must be [N, O, OH*OW] for this geometry, got "
                           f"{tuple(grad_output.shape)} expected L={Lc}")
    return _lre_grads(grad_output, xc, w, dx, dw, g, N, K, Lc, O)


# --------------------------------------------------------- custom backward
def custom_grads(operand, wq: Tensor, dy: Tensor, dx_lut, dw_lut, N: int, K: int, Lc: int,
                 mask_w=None, scale_w=None, wbase=None, dy_scale=None, img_ste=None,
                 w_zero_point=None):
    """(grad_x [N,K,L] or None, grad_w [O,K] or None) of the pair-table
    estimator from the LUT GEMM's row-offset operand (xt, Rpad) and the uint8
    weight index image wq [O,K]; dx_lut / dw_lut are fp32 [65536] tables
    indexed [x*256 + w] (None skips that gradient).  mask_w / scale_w fuse
    the per-channel weight fake-quant STE into grad_w.  wbase: the caller
    guarantees every index of wq lies in [wbase, wbase + 16) (weight_bits <=
    4), and grad_x runs on the matrix cores (atx_custom_grad_dx_narrow).
    dy_scale [O] (optional): the gradients of dy * dy_scale[o], with no scaled
    copy of dy where the kernels take the factor.
    img_ste (with wbase; a 1x1 stride-1 unpadded conv, whose column gradient
    is the image gradient): (pos [N, L] or None, mask [N, K, L] or None,
    scale [1]) -- grad_x comes back as col2im(grad_x, pos, mask, scale) of
    that geometry, computed in the grad_x kernel's epilogue.
    w_zero_point = (go_sum [O], scale_x [1], zero_x [1]), with scale_w: the
    uint8 layer's weight zero-point term, grad_w -= (go_sum * (scale_x *
    scale_w)) * zero_x before the STE (atx_custom_grad_dw_uint8)."""
    xt, Rpad = operand
    O = wq.size(0)
    dyc = dy.contiguous()
    if dyc.dtype != torch.float32 or tuple(dyc.shape) != (N, O, Lc):
        raise RuntimeError(f"dY must be float32 of shape {(N, O, Lc)}")
    if dy_scale is not None:
        dy_scale = dy_scale.contiguous()
        if dy_scale.dtype != torch.float32 or dy_scale.numel() != O or \
                dy_scale.device != dyc.device:
            raise RuntimeError(f"dy_scale must be float32 [{O}] on {dyc.device}")
    _, wt, Opad = _pack_w(wq.contiguous(), 0)
    dev, s = dyc.device, L.stream_of(dyc)
    gx = gw = None
    if dx_lut is not None:
        tab = lut_image(dx_lut)[1]
        gx = torch.empty((N, K, Lc), dtype=torch.float32, device=dev)
        if wbase is not None:
            dyx, dsx = dyc, dy_scale
            if dy_scale is not None and O > 4096:   # the kernel holds at most 4096 factors
                dyx, dsx = dyc * dy_scale.view(1, -1, 1), None
            if img_ste is not None:
                pos, mask, scale = img_ste
                pos = None if pos is None else pos.contiguous()
                mask = None if mask is None else mask.contiguous()
                if mask is not None and (mask.dtype != torch.bool or mask.numel() != N * K * Lc):
                    raise RuntimeError(f"mask must be bool with {N * K * Lc} elements")
                if pos is not None and (pos.dtype != torch.float32 or pos.numel() != N * Lc):
                    raise RuntimeError(f"pos must be float32 with {N * Lc} elements")
                L.call("atx_custom_grad_dx_narrow_img", L.ptr(xt), Rpad, L.ptr(wt), Opad,
                       L.ptr(dyx), L.ptr(dsx), L.ptr(tab), int(wbase), N, K, Lc, O, L.ptr(pos),
                       L.ptr(mask), L.ptr(None if scale is None else scale.contiguous()),
                       L.ptr(gx), s)
            else:
                L.call("atx_custom_grad_dx_narrow", L.ptr(xt), Rpad, L.ptr(wt), Opad,
                       L.ptr(dyx), L.ptr(dsx), L.ptr(tab), int(wbase), N, K, Lc, O, L.ptr(gx), s)
        else:
            dyx = dyc if dy_scale is None else dyc * dy_scale.view(1, -1, 1)
            L.call("atx_custom_grad_dx", L.ptr(xt), Rpad, L.ptr(wt), Opad, L.ptr(dyx),
                   L.ptr(tab), N, K, Lc, O, L.ptr(gx), s)
    if dw_lut is not None:
        tab = lut_image(dw_lut)[1]
        gw = torch.empty((O, K), dtype=torch.float32, device=dev)
        wsb = L.query("atx_custom_grad_dw_workspace_bytes", N, K, Lc, O)
        ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=dev)
        if w_zero_point is None:
            L.call("atx_custom_grad_dw", L.ptr(xt), Rpad, L.ptr(wt), Opad, L.ptr(dyc),
                   L.ptr(dy_scale), L.ptr(tab), N, K, Lc, O, L.ptr(mask_w), L.ptr(scale_w),
                   L.ptr(gw), L.ptr(ws), s)
        else:
            zsum, zsx, zzx = (t.contiguous() for t in w_zero_point)
            for name, t, n in (("go_sum", zsum, O), ("scale_x", zsx, 1), ("zero_x", zzx, 1)):
                if t.dtype != torch.float32 or t.numel() != n or t.device != dev:
                    raise RuntimeError(f"{name} must be float32 [{n}] on {dev}")
            if scale_w is None:
                raise RuntimeError("w_zero_point needs scale_w")
            L.call("atx_custom_grad_dw_uint8", L.ptr(xt), Rpad, L.ptr(wt), Opad, L.ptr(dyc),
                   L.ptr(dy_scale), L.ptr(tab), N, K, Lc, O, L.ptr(mask_w), L.ptr(scale_w),
                   L.ptr(zsum), L.ptr(zsx), L.ptr(zzx), L.ptr(gw), L.ptr(ws), s)
    return gx, gw


def pack_rows_u8(X: Tensor):
    """Row-offset operand (xt, Rpad) of a uint8 index image X [N,K,L]."""
    Xc = X.contiguous()
    N, K, Lc = Xc.shape
    Rpad = L.round_up(max(N * Lc, 1), L.ROW_TILE)
    xt = torch.empty((L.operand_rows(K), Rpad), dtype=torch.int16, device=Xc.device)
    L.call("atx_pack_x_u8", L.ptr(Xc), N, K, Lc, L.ptr(xt), Rpad, None, L.stream_of(Xc))
    return xt, Rpad


def _custom(kind, X, W, dY, lut, signed):
    """The reference's op-level custom-gradient kernels: X [N,K,L], W [O,K]
    uint8 LUT indices (or int8 values, index v+128), dY [N,O,L] fp32."""
    want = torch.int8 if signed else torch.uint8
    for t, nm in ((X, "X"), (W, "W"), (dY, "dY"), (lut, "lut")):
        if not t.is_cuda:
            raise RuntimeError(f"{nm} must be a CUDA tensor")
    if X.dtype != want or W.dtype != want:
        raise RuntimeError(f"X and W must be {want}")
    if dY.dtype != torch.float32 or lut.dtype != torch.float32 or lut.numel() != 65536:
        raise RuntimeError("dY must be float32 and lut a float32 [65536] table")
    if X.dim() != 3 or W.dim() != 2 or dY.dim() != 3:
        raise RuntimeError("expected X [N,K,L], W [O,K], dY [N,O,L]")
    N, K, Lc = X.shape
    O = W.size(0)
    if W.size(1) != K or tuple(dY.shape) != (N, O, Lc):
        raise RuntimeError("shape mismatch between X, W and dY")
    if signed:
        X = (X.to(torch.int16) + 128).to(torch.uint8)
        W = (W.to(torch.int16) + 128).to(torch.uint8)
    gx, gw = custom_grads(pack_rows_u8(X), W, dY, lut if kind == "dx" else None,
                          lut if kind == "dw" else None, N, K, Lc)
    return gx if kind == "dx" else gw


def bgemm_custom_grad_uint8_dx(X, W, dY, dx_lut):
    """csrc/cuda/bgemm_custom_grad_optimize.cu:212-256 (uint8 LUT indices)."""
    return _custom("dx", X, W, dY, dx_lut, False)


def bgemm_custom_grad_uint8_dw(X, W, dY, dW_lut):
    """csrc/cuda/bgemm_custom_grad_optimize.cu:259-301."""
    return _custom("dw", X, W, dY, dW_lut, False)


def bgemm_custom_grad_int8_dx(X, W, dY, dx_lut):
    """csrc/cuda/bgemm_custom_grad_optimize.cu:497-541 (int8 values, index v+128)."""
    return _custom("dx", X, W, dY, dx_lut, True)


def bgemm_custom_grad_int8_dw(X, W, dY, dW_lut):
    """csrc/cuda/bgemm_custom_grad_optimize.cu:544-585."""
    return _custom("dw", X, W, dY, dW_lut, True)


# ------------------------------------------------------------- fake-quant
def _reduce_ws(dev):
    return torch.empty(L.query("atx_reduce_workspace_bytes") // 4, dtype=torch.float32,
                       device=dev)


def require_cuda_f32(t: Tensor, name: str):
    """The reference's TORCH_CHECK(x.is_cuda() / scalar_type() == kFloat32)
    (csrc/claude/quantization.cu:190-193): the kernels read fp32 device memory."""
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32, got {t.dtype}")


# activation dtypes the *_dt kernels read besides fp32
LOWP = {torch.float16: L.ATX_DT_F16, torch.bfloat16: L.ATX_DT_BF16}


def dtype_code(t: Tensor) -> int:
    """ATX_DT_* code of an fp32 / fp16 / bf16 tensor."""
    if t.dtype == torch.float32:
        return L.ATX_DT_F32
    if t.dtype in LOWP:
        return LOWP[t.dtype]
    raise RuntimeError(f"expected a float32, float16 or bfloat16 tensor, got {t.dtype}")


def require_cuda_float(t: Tensor, name: str):
    """A CUDA tensor of fp32, fp16 or bf16 (the activation dtypes the
    statistic and fake-quant kernels read)."""
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"{name} must be float32, float16 or bfloat16, got {t.dtype}")


def require_param(p, x: Tensor, name: str, numel: int = 1):
    """A scale / zero-point operand: fp32, `numel` elements, on x's device
    (csrc/claude/quantization.cu:190-193,269-274)."""
    if p is None:
        return
    if not p.is_cuda or p.device != x.device:
        raise RuntimeError(f"{name} must be a CUDA tensor on {x.device}")
    if p.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32, got {p.dtype}")
    if p.numel() != numel:
        what = "a scalar tensor" if numel == 1 else f"a tensor of {numel} elements"
        raise RuntimeError(f"{name} must be {what}, got {p.numel()} elements")


def fakequant_per_tensor(x: Tensor, scale: Tensor, qmin: int, qmax: int, zero_point=None,
                         want_q=True, q8_dtype=None, nonneg=None):
    """(q, mask bool[, q8]) of the fused per-tensor fake-quant
    (csrc/claude/quantization.cu:187-221 symmetric, 260-311 asymmetric); q
    has x's dtype.  An fp16 / bf16 x takes the reference's unfused statements
    in that dtype (nn/quantization.py:44-52,72-80; atx_fakequant_fwd_dt).
    nonneg: optional device int32 flag (upper_flag()), cleared when some
    quantized value is negative."""
    require_cuda_float(x, "x")
    require_param(scale, x, "scale")
    require_param(zero_point, x, "zero_point")
    if qmin >= qmax:
        raise RuntimeError(f"qmin must be < qmax, got [{qmin}, {qmax}]")
    xc = x.contiguous()
    q = torch.empty_like(xc) if want_q else None
    mask = torch.empty(xc.shape, dtype=torch.bool, device=xc.device)
    q8 = torch.empty(xc.shape, dtype=q8_dtype, device=xc.device) if q8_dtype else None
    zp = L.ptr(None if zero_point is None else zero_point.contiguous())
    if xc.dtype in LOWP:
        L.call("atx_fakequant_fwd_dt", L.ptr(xc), LOWP[xc.dtype], xc.numel(),
               L.ptr(scale.contiguous()), zp, qmin, qmax, L.ptr(q), L.ptr(mask), L.ptr(q8),
               L.ptr(nonneg), L.stream_of(xc))
    else:
        L.call("atx_fakequant_fwd", L.ptr(xc), xc.numel(), L.ptr(scale.contiguous()), zp, qmin,
               qmax, L.ptr(q), L.ptr(mask), L.ptr(q8), L.ptr(nonneg), L.stream_of(xc))
    return q, mask, q8


def fakequant_rows(x: Tensor, scale: Tensor, qmin: int, qmax: int, offset: int,
                   zero_point=None, upper=None):
    """Input fake-quant of a 1x1, stride-1, unpadded conv fused with its
    operand packing: x [N,K,H,W] -> (mask bool [N,K,H,W], (xt, Rpad)), the
    row-offset operand that fakequant_per_tensor's byte image would give
    through conv_forward's im2col (offset 128: int8 image, 0: uint8).
    upper: optional device int32 flag (upper_flag()), cleared when some LUT
    index of the operand is below 128."""
    require_cuda_f32(x, "x")
    require_param(scale, x, "scale")
    require_param(zero_point, x, "zero_point")
    if x.dim() < 2:
        raise RuntimeError(f"x must have at least 2 dimensions [N, C, ...], got {x.dim()}")
    if qmin >= qmax:
        raise RuntimeError(f"qmin must be < qmax, got [{qmin}, {qmax}]")
    xc = x.contiguous()
    N, K = xc.size(0), xc.size(1)
    Lc = xc.numel() // max(N * K, 1)
    Rpad = L.round_up(max(N * Lc, 1), L.ROW_TILE)
    mask = torch.empty(xc.shape, dtype=torch.bool, device=xc.device)
    xt = torch.empty((L.operand_rows(K), Rpad), dtype=torch.int16, device=xc.device)
    L.call("atx_fakequant_rows", L.ptr(xc), N, K, Lc, L.ptr(scale.contiguous()),
           L.ptr(None if zero_point is None else zero_point.contiguous()), qmin, qmax, offset,
           L.ptr(mask), L.ptr(xt), Rpad, L.ptr(upper), L.stream_of(xc))
    return mask, (xt, Rpad)


def conv_forward_rows(xt_rpad, w_idx_or_val: Tensor, lut: Tensor, g, offset: int,
                      out_kind=L.ATX_OUT_F32, sx=None, sw=None, bias=None, packed_w=None,
                      wbase=None, x_upper=None):
    """LUT conv from a prepacked row-offset operand (xt, Rpad) of geometry g
    (fakequant_rows, or conv_forward's return_operand): (y, wq).  wbase and
    x_upper as in conv_forward."""
    xt, Rpad = xt_rpad
    N, K = g.N, g.C * g.KH * g.KW
    Lc = g.OH * g.OW
    O = w_idx_or_val.size(0)
    if w_idx_or_val.size(1) != K:
        raise RuntimeError(f"weight has {w_idx_or_val.size(1)} taps, geometry needs {K}")
    if xt.size(0) != L.operand_rows(K) or Rpad < N * Lc or xt.size(1) != Rpad:
        raise RuntimeError(f"operand {tuple(xt.shape)} does not match K={K}, rows={N * Lc}")
    if packed_w is None:
        wq, wt, Opad = _pack_w(w_idx_or_val.contiguous(), offset)
    else:
        wq, wt, Opad = packed_w
    ydt = torch.int32 if out_kind == L.ATX_OUT_I32 else torch.float32
    y = torch.empty((N, O, Lc), dtype=ydt, device=xt.device)
    _gemm(xt, Rpad, wt, Opad, N, K, Lc, O, lut, out_kind, y, sx, sw, bias, wbase=wbase,
          x_upper=x_upper)
    return y, wq


def fakequant_per_tensor_backward(grad_output: Tensor, mask: Tensor, scale: Tensor,
                                  channels: int = 1, inner: int = 1, dtype=None) -> Tensor:
    """gx = (mask ? go : 0) / max(scale, 1e-12) (csrc/claude/quantization.cu:223-258);
    scale has one element, or `channels` for a per-channel mask of
    channels x inner elements.  dtype (default: grad_output's) fp16 / bf16:
    the per-tensor gradient of an x of that dtype, go * mask / s in it
    (nn/quantization.py:58-62; grad_output fp32 or that dtype,
    atx_fakequant_bwd_dt)."""
    dtype = grad_output.dtype if dtype is None else dtype
    if dtype in LOWP:
        if not grad_output.is_cuda or grad_output.dtype not in (torch.float32, dtype):
            raise RuntimeError(f"grad_output must be a CUDA float32 or {dtype} tensor")
        if mask.dtype != torch.bool or mask.device != grad_output.device or \
                mask.shape != grad_output.shape:
            raise RuntimeError("mask must be a bool CUDA tensor of grad_output's shape")
        if channels != 1:
            raise RuntimeError("fp16 / bf16 fake-quant gradients are per tensor")
        require_param(scale, grad_output, "scale")
        go = grad_output.contiguous()
        gx = torch.empty(go.shape, dtype=dtype, device=go.device)
        L.call("atx_fakequant_bwd_dt", L.ptr(go), dtype_code(go), L.ptr(mask.contiguous()),
               go.numel(), L.ptr(scale.contiguous()), LOWP[dtype], L.ptr(gx), L.stream_of(go))
        return gx
    require_cuda_f32(grad_output, "grad_output")
    if not mask.is_cuda or mask.device != grad_output.device:
        raise RuntimeError(f"mask must be a CUDA tensor on {grad_output.device}")
    if mask.dtype != torch.bool:
        raise RuntimeError(f"mask must be bool, got {mask.dtype}")
    if grad_output.shape != mask.shape:
        raise RuntimeError(f"grad_output/mask shape mismatch: {tuple(grad_output.shape)} vs "
                           f"{tuple(mask.shape)}")
    require_param(scale, grad_output, "scale", channels)
    if channels != 1 and channels * inner != grad_output.numel():
        raise RuntimeError(f"{channels} channels x {inner} do not cover "
                           f"{grad_output.numel()} elements")
    go = grad_output.contiguous()
    gx = torch.empty_like(go)
    L.call("atx_fakequant_bwd", L.ptr(go), L.ptr(mask.contiguous()), go.numel(),
           L.ptr(scale.contiguous()), channels, inner, L.ptr(gx), L.stream_of(go))
    return gx


def fakequant_per_channel(w: Tensor, scale: Tensor, qmin: int, qmax: int, zero_point=None,
                          offset=None, want_wt=False, want_q=True):
    """Per-channel (axis 0) fake-quant of a weight: (q or None, mask, wq index
    image, wt GEMM operand or None, Opad)."""
    require_cuda_f32(w, "w")
    if w.dim() < 1:
        raise RuntimeError("w must have a channel dimension")
    O = w.size(0)
    require_param(scale, w, "scale", O)
    require_param(zero_point, w, "zero_point", O)
    if qmin >= qmax:
        raise RuntimeError(f"qmin must be < qmax, got [{qmin}, {qmax}]")
    wc = w.contiguous()
    inner = wc.numel() // max(O, 1)
    q = torch.empty_like(wc) if want_q else None
    mask = torch.empty(wc.shape, dtype=torch.bool, device=wc.device)
    wq = torch.empty((O, inner), dtype=torch.uint8, device=wc.device) if offset is not None \
        else None
    Opad = L.round_up(max(O, 1), L.COL_TILE)
    wt = torch.empty((inner, Opad), dtype=torch.uint8, device=wc.device) if want_wt else None
    L.call("atx_fakequant_channel_fwd", L.ptr(wc), O, inner, L.ptr(scale.contiguous()),
           L.ptr(None if zero_point is None else zero_point.contiguous()), qmin, qmax,
           offset if offset is not None else 0, L.ptr(q), L.ptr(mask), L.ptr(wq), L.ptr(wt),
           Opad, L.stream_of(wc))
    return q, mask, wq, wt, Opad
