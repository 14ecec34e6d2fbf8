"""ctypes binding of libatx.so, the C ABI declared in include/atx.h.

The library is loaded once, after torch (so it shares torch's HIP runtime:
both runtimes carry the SONAME libamdhip64.so.7 and the dynamic linker reuses
the one torch already mapped).  Every call returns an int status; a non-zero
status raises RuntimeError carrying atx_last_error().  There is no fallback:
if the library is missing, the product path fails loudly.
"""
import ctypes
import os

import torch  # noqa: F401  (must be imported before libatx is loaded)

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libatx.so")

c_int, c_ll, c_float, c_vp = ctypes.c_int, ctypes.c_longlong, ctypes.c_float, ctypes.c_void_p

ATX_LUT_I16, ATX_LUT_U16, ATX_LUT_F32 = 0, 1, 2
ATX_OUT_F32, ATX_OUT_I32, ATX_OUT_DEQUANT = 0, 1, 2
ATX_DT_F32, ATX_DT_F16, ATX_DT_BF16 = 0, 1, 2
ROW_TILE, COL_TILE = 2048, 32
NOALLOC_SCRATCH_BYTES = 64 << 20     # ATX_NOALLOC_SCRATCH_BYTES


class ConvGeom(ctypes.Structure):
    _fields_ = [(n, c_int) for n in
                ("N", "C", "H", "W", "KH", "KW", "SH", "SW", "PH", "PW", "DH", "DW",
                 "OH", "OW")]


ABI_VERSION = 2                      # ATX_ABI_VERSION


class GemmEpilogue(ctypes.Structure):
    """atx_gemm_epilogue; `size` (the first field) is filled in."""
    _fields_ = [("size", c_int), ("out_kind", c_int), ("scale_x", c_vp), ("scale_w", c_vp),
                ("bias", c_vp), ("x_upper", c_vp)]

    def __init__(self, out_kind=0, scale_x=None, scale_w=None, bias=None, x_upper=None):
        super().__init__(ctypes.sizeof(GemmEpilogue), out_kind, scale_x, scale_w, bias, x_upper)


# name -> (restype, argtypes); mirrors include/atx.h one to one.
_SIGS = {
    "atx_last_error": (ctypes.c_char_p, []),
    "atx_version": (c_int, []),
    "atx_set_timing_events": (c_int, [c_vp, c_vp]),
    "atx_lut_prepare": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp]),
    "atx_pack_x_f32": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_vp, c_vp, c_int, c_vp, c_vp]),
    "atx_pack_x_u8": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp, c_vp]),
    "atx_pack_w_f32": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_vp, c_int, c_vp]),
    "atx_pack_w_u8": (c_int, [c_vp, c_int, c_int, c_vp, c_int, c_vp]),
    "atx_im2col_rows": (c_int, [c_vp, c_int, ConvGeom, c_int, c_vp, c_vp, c_int, c_vp]),
    "atx_im2col_u8": (c_int, [c_vp, c_int, ConvGeom, c_vp, c_vp]),
    "atx_lut_gemm_workspace_bytes": (c_ll, [c_int, c_int, c_int, c_int]),
    "atx_lut_gemm": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp,
                             c_vp, c_int, GemmEpilogue, c_vp, c_vp, c_vp]),
    "atx_lut_gemm_noalloc": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_int,
                                     c_vp, c_vp, c_int, GemmEpilogue, c_vp, c_vp]),
    "atx_lut_gemm_narrow_workspace_bytes": (c_ll, [c_int, c_int, c_int, c_int]),
    "atx_lut_gemm_narrow": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp,
                                    c_int, c_int, GemmEpilogue, c_vp, c_vp, c_vp]),
    "atx_lut_gemm_narrow_uint8": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_int,
                                          c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                          c_vp, c_vp, c_vp]),
    "atx_fakequant_fwd": (c_int, [c_vp, c_ll, c_vp, c_vp, c_int, c_int, c_vp, c_vp, c_vp,
                                  c_vp, c_vp]),
    "atx_fakequant_rows": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_vp, c_int, c_int, c_int,
                                   c_vp, c_vp, c_int, c_vp, c_vp]),
    "atx_fakequant_bwd": (c_int, [c_vp, c_vp, c_ll, c_vp, c_int, c_ll, c_vp, c_vp]),
    "atx_fakequant_channel_fwd": (c_int, [c_vp, c_int, c_ll, c_vp, c_vp, c_int, c_int, c_int,
                                          c_vp, c_vp, c_vp, c_vp, c_int, c_vp]),
    "atx_col2im": (c_int, [c_vp, ConvGeom, c_vp, c_vp, c_vp, c_vp]),
    "atx_col2im_pos": (c_int, [c_vp, ConvGeom, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "atx_tap_sum_workspace_bytes": (c_ll, [ConvGeom]),
    "atx_tap_sum": (c_int, [c_vp, c_int, ConvGeom, c_vp, c_vp, c_vp, c_vp]),
    "atx_zero_point_pos": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "atx_zero_point_terms_workspace_bytes": (c_ll, [c_int, c_int, c_int]),
    "atx_zero_point_terms": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp,
                                     c_vp, c_vp]),
    "atx_tap_sum_bwd": (c_int, [c_vp, ConvGeom, c_vp, c_vp]),
    "atx_uint8_dequant": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                  c_vp, c_int, c_vp]),
    "atx_reduce_workspace_bytes": (c_ll, []),
    "atx_absmax": (c_int, [c_vp, c_ll, c_vp, c_vp, c_vp]),
    "atx_minmax": (c_int, [c_vp, c_ll, c_vp, c_vp, c_vp, c_vp]),
    "atx_ema_absmax_apply": (c_int, [c_vp, c_float, c_float, c_float, c_vp, c_vp]),
    "atx_absmax_ema": (c_int, [c_vp, c_ll, c_vp, c_vp, c_float, c_float, c_float, c_vp, c_vp]),
    "atx_absmax_ema_upper": (c_int, [c_vp, c_ll, c_vp, c_vp, c_float, c_float, c_float, c_vp,
                                     c_vp, c_vp]),
    "atx_absmax_dt": (c_int, [c_vp, c_int, c_ll, c_vp, c_vp, c_vp]),
    "atx_ema_absmax_apply_dt": (c_int, [c_vp, c_int, c_float, c_float, c_float, c_vp, c_vp]),
    "atx_absmax_ema_upper_dt": (c_int, [c_vp, c_int, c_ll, c_vp, c_vp, c_float, c_float,
                                        c_float, c_vp, c_vp, c_vp]),
    "atx_fakequant_fwd_dt": (c_int, [c_vp, c_int, c_ll, c_vp, c_vp, c_int, c_int, c_vp, c_vp,
                                     c_vp, c_vp, c_vp]),
    "atx_fakequant_bwd_dt": (c_int, [c_vp, c_int, c_vp, c_ll, c_vp, c_int, c_vp, c_vp]),
    "atx_weight_scale_ema_dt": (c_int, [c_vp, c_int, c_int, c_ll, c_float, c_float, c_float,
                                        c_int, c_vp, c_vp]),
    "atx_minmax_ema": (c_int, [c_vp, c_ll, c_vp, c_vp, c_vp, c_float, c_float, c_int, c_vp,
                               c_vp, c_vp, c_vp, c_vp]),
    "atx_ema_minmax_apply": (c_int, [c_vp, c_vp, c_float, c_float, c_int, c_vp, c_vp, c_vp,
                                     c_vp, c_vp]),
    "atx_weight_scale_ema": (c_int, [c_vp, c_int, c_ll, c_float, c_float, c_float, c_int,
                                     c_vp, c_vp]),
    "atx_weight_minmax_ema": (c_int, [c_vp, c_int, c_ll, c_float, c_float, c_int, c_vp, c_vp,
                                      c_vp, c_vp, c_vp]),
    "atx_lut_map": (c_int, [c_vp, c_int, c_ll, c_vp, c_vp, c_vp]),
    "atx_lut_map_pad": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_vp,
                                c_vp, c_vp]),
    "atx_conv_bwd_data_col": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp,
                                      c_vp]),
    "atx_pack_rows_strided": (c_int, [c_vp, c_int, c_int, c_int, c_ll, c_ll, c_int, c_vp, c_vp,
                                      c_int, c_vp, c_vp]),
    "atx_pack_cols_strided": (c_int, [c_vp, c_int, c_int, c_int, c_ll, c_ll, c_int, c_vp, c_vp,
                                      c_int, c_vp]),
    "atx_parse_text_table": (c_int, [ctypes.c_char_p, c_int, c_vp, c_ll, c_vp]),
    "atx_lre_tables": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp]),
    "atx_date_tables": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp]),
    "atx_dwconv_fwd": (c_int, [c_vp, c_int, ConvGeom, c_int, c_vp, c_vp, c_vp, c_int,
                               GemmEpilogue, c_vp, c_vp]),
    "atx_dwconv_bwd_data": (c_int, [c_vp, c_vp, c_vp, ConvGeom, c_vp, c_vp, c_vp, c_vp, c_vp,
                                    c_vp]),
    "atx_dwconv_bwd_weight_workspace_bytes": (c_ll, [ConvGeom]),
    "atx_dwconv_bwd_weight": (c_int, [c_vp, c_vp, c_int, ConvGeom, c_int, c_vp, c_vp, c_vp,
                                      c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "atx_conv_bwd_data_workspace_bytes": (c_ll, [ConvGeom, c_int]),
    "atx_conv_bwd_data": (c_int, [c_vp, c_vp, c_vp, ConvGeom, c_int, c_vp, c_vp, c_vp, c_vp,
                                  c_vp, c_vp, c_vp]),
    "atx_conv_bwd_weight_workspace_bytes": (c_ll, [c_int, c_int, c_ll]),
    "atx_conv_bwd_weight_rows": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp,
                                         c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "atx_conv_bwd_weight": (c_int, [c_vp, c_vp, c_int, ConvGeom, c_int, c_int, c_vp, c_vp,
                                    c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "atx_custom_grad_dx": (c_int, [c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_int, c_int, c_int,
                                   c_int, c_vp, c_vp]),
    "atx_custom_grad_dx_narrow": (c_int, [c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_int,
                                          c_int, c_int, c_int, c_int, c_vp, c_vp]),
    "atx_custom_grad_dx_narrow_img": (c_int, [c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_int,
                                              c_int, c_int, c_int, c_int, c_vp, c_vp, c_vp,
                                              c_vp, c_vp]),
    "atx_custom_grad_dw_workspace_bytes": (c_ll, [c_int, c_int, c_int, c_int]),
    "atx_custom_grad_dw": (c_int, [c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_int, c_int,
                                   c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "atx_custom_grad_dw_uint8": (c_int, [c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_int,
                                         c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp,
                                         c_vp, c_vp, c_vp]),
}

_lib = None


def load():
    """Loads libatx.so (once) and declares every entry point's signature."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`"
                " (the HIP extension is required, there is no fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.atx_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} implements ABI version {lib.atx_version()}, this "
                               f"binding needs {ABI_VERSION}; rebuild the library")
        _lib = lib
    return _lib


def exported_symbols():
    return sorted(_SIGS)


def call(name, *args):
    """Calls an int-returning entry point; raises RuntimeError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.atx_last_error().decode(errors="replace")
        kind = {-1: "invalid argument", -2: "launch failure", -3: "out of range"}.get(rc, rc)
        raise RuntimeError(f"{name} failed ({kind}): {msg}")


def query(name, *args):
    """Calls a value-returning entry point (sizes, versions)."""
    return getattr(load(), name)(*args)


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream_of(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def geom(N, C, H, W, KH, KW, SH, SW, PH, PW, DH, DW):
    OH = (H + 2 * PH - DH * (KH - 1) - 1) // SH + 1
    OW = (W + 2 * PW - DW * (KW - 1) - 1) // SW + 1
    return ConvGeom(N, C, H, W, KH, KW, SH, SW, PH, PW, DH, DW, OH, OW)


def round_up(v, m):
    return (v + m - 1) // m * m


def operand_rows(K):
    """k-rows of the LUT GEMM's row-offset operand: K rounded up to a quad."""
    return round_up(K, 4)
