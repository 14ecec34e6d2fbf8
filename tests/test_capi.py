"""libatx.so loads on the CPU, exports every symbol include/atx.h declares, and
its host-side argument validation returns error codes without touching a GPU."""
import ctypes
import os
import re

import pytest

from approxtorch_amd.backend import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions(name="atx.h"):
    text = open(os.path.join(ROOT, "include", name)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^(?:int|long long|const char\*)\s+(atx_\w+)\(", text, flags=re.M)


def test_every_declared_symbol_is_exported_and_bound():
    lib = L.load()
    names = header_functions()
    assert len(names) >= 30
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(names) == L.exported_symbols()
    assert lib.atx_version() == L.ABI_VERSION == 2


def test_diag_probes_live_in_their_own_library():
    """The measurement probes (include/atx_diag.h) are exported by
    libatx_diag.so and not by the product library."""
    diag = ctypes.CDLL(os.path.join(ROOT, "approxtorch_amd", "libatx_diag.so"))
    lib = L.load()
    names = header_functions("atx_diag.h")
    assert sorted(names) == ["atx_inner_probe", "atx_lds_probe", "atx_valu_probe"]
    for n in names:
        assert hasattr(diag, n) and not hasattr(lib, n), n


def test_invalid_arguments_return_einval_without_gpu():
    lib = L.load()
    ep = L.GemmEpilogue(0, None, None, None)
    rc = lib.atx_lut_gemm(None, 1024, None, 64, -1, 4, 4, 4, None, None, 0, ep, None, None, None)
    assert rc == -1
    assert b"negative size" in lib.atx_last_error()
    rc = lib.atx_lut_gemm(None, 100, None, 64, 1, 4, 4, 4, None, None, 0, ep, None, None, None)
    assert rc == -1 and b"Rpad" in lib.atx_last_error()
    rc = lib.atx_fakequant_fwd(None, 10, None, None, 5, 5, None, None, None, None, None)
    assert rc == -1 and b"qmin" in lib.atx_last_error()
    g = L.geom(1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 1, 1)
    g.OH = 7
    rc = lib.atx_im2col_u8(None, 0, g, None, None)
    assert rc == -1 and b"OH/OW" in lib.atx_last_error()


def test_epilogue_of_another_abi_is_rejected_without_gpu():
    """A caller built against the version-1 header passes a struct whose
    first field is out_kind (0..2): rejected on the host, nothing launched."""
    lib = L.load()

    class EpilogueV1(ctypes.Structure):
        _fields_ = [("out_kind", ctypes.c_int), ("scale_x", ctypes.c_void_p),
                    ("scale_w", ctypes.c_void_p), ("bias", ctypes.c_void_p)]

    assert ctypes.sizeof(L.GemmEpilogue) == 40 and L.GemmEpilogue(2).size == 40
    for name, args in (("atx_lut_gemm", (None, 2048, None, 32, 1, 4, 4, 4, None, None, 0)),
                       ("atx_lut_gemm_narrow", (None, 2048, None, 32, 1, 4, 4, 4, None, 0, 0))):
        fn = ctypes.CDLL(L.LIB_PATH)[name]          # unprototyped: any struct goes through
        fn.restype = ctypes.c_int
        old = EpilogueV1(2, None, None, None)
        rc = fn(*[ctypes.c_void_p(a) if a is None else ctypes.c_int(a) for a in args], old,
                None, None, None)
        assert rc == -1, name
        assert b"atx_gemm_epilogue.size" in lib.atx_last_error(), name
    bad = L.GemmEpilogue(0)
    bad.size = 32
    rc = lib.atx_lut_gemm(None, 2048, None, 32, 1, 4, 4, 4, None, None, 0, bad, None, None, None)
    assert rc == -1 and b"expected 40" in lib.atx_last_error()


def test_pack_w_needs_an_output_without_gpu():
    """atx_pack_w_f32 writes wq, wt or both; with neither it fails on the
    host before launching anything."""
    lib = L.load()
    rc = lib.atx_pack_w_f32(None, 4, 9, 128, None, None, 32, None)
    assert rc == -1 and b"null pointer" in lib.atx_last_error()


def test_workspace_queries_are_host_only():
    assert L.query("atx_lut_gemm_workspace_bytes", 32, 2304, 4096, 256) == 0      # 512 tiles
    assert L.query("atx_lut_gemm_workspace_bytes", 8, 576, 1024, 64) > 0          # split-K
    assert L.query("atx_lut_gemm_workspace_bytes", 1, 40000, 49, 64) > 0          # K > int32 bound
    assert L.query("atx_reduce_workspace_bytes") == 1024 * 8


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        L.load()


def header_arities(name="atx.h"):
    """name -> number of parameters of every function include/<name> declares."""
    text = open(os.path.join(ROOT, "include", name)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^(?:int|long long|const char\*)\s+(atx_\w+)\(([^)]*)\)", text,
                         flags=re.M | re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_binding_arities_match_the_header():
    """Every ctypes signature in backend/_lib.py has as many parameters as the
    header's declaration (a missing slot would pass the stream as an int)."""
    arity = header_arities()
    for name, (_, args) in L._SIGS.items():
        assert len(args) == arity[name], (name, len(args), arity[name])
