"""atx_lut_gemm_noalloc (the LUT GEMM with a library-owned static scratch
buffer instead of a caller workspace) against atx_lut_gemm, through the C
ABI: bit-exact int32 sums and identical dequantized outputs, on consecutive
calls whose schedules use the scratch (stream-K slots, then split-K
partials of a smaller problem, then whole tiles)."""
import ctypes

import numpy as np
import pytest
import torch

from approxtorch_amd.backend import _lib as L
from approxtorch_amd.backend import ops

DEV = "cuda"


def _operands(seed, N, K, Lc, Oc):
    r = np.random.default_rng(seed)
    xi = torch.as_tensor(r.integers(0, 256, (N, K, Lc), dtype=np.uint8), device=DEV)
    wi = torch.as_tensor(r.integers(0, 256, (Oc, K), dtype=np.uint8), device=DEV)
    Rpad = L.round_up(max(N * Lc, 1), L.ROW_TILE)
    Opad = L.round_up(max(Oc, 1), L.COL_TILE)
    xt = torch.empty((L.operand_rows(K), Rpad), dtype=torch.int16, device=DEV)
    wt = torch.empty((K, Opad), dtype=torch.uint8, device=DEV)
    s = L.stream_of(xi)
    L.call("atx_pack_x_u8", xi.data_ptr(), N, K, Lc, xt.data_ptr(), Rpad, None, s)
    L.call("atx_pack_w_u8", wi.data_ptr(), Oc, K, wt.data_ptr(), Opad, s)
    sw = torch.as_tensor(r.random(Oc).astype(np.float32) + 0.01, device=DEV)
    sx = torch.tensor(0.0173, device=DEV)
    bias = torch.as_tensor(r.standard_normal(Oc).astype(np.float32), device=DEV)
    return xt, Rpad, wt, Opad, sx, sw, bias


def _lut(seed):
    r = np.random.default_rng(seed)
    a = np.arange(256) - 128
    p = a[:, None] * a[None, :]
    e = np.rint(r.normal(0, 1, p.shape) * (0.02 * np.abs(p) + 1))
    return torch.as_tensor(np.clip(p + e, -32768, 32767).astype(np.float32).reshape(-1),
                           device=DEV)


def _run(N, K, Lc, Oc, seed, out_kind):
    xt, Rpad, wt, Opad, sx, sw, bias = _operands(seed, N, K, Lc, Oc)
    img16, imgf, cls = ops.lut_image(_lut(seed))
    ydt = torch.int32 if out_kind == L.ATX_OUT_I32 else torch.float32
    ep = L.GemmEpilogue(out_kind, sx.data_ptr(), sw.data_ptr(), bias.data_ptr())
    s = L.stream_of(xt)
    y_ref = torch.empty((N, Oc, Lc), dtype=ydt, device=DEV)
    wsb = L.query("atx_lut_gemm_workspace_bytes", N, K, Lc, Oc)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.int32, device=DEV)
    L.call("atx_lut_gemm", xt.data_ptr(), Rpad, wt.data_ptr(), Opad, N, K, Lc, Oc,
           img16.data_ptr(), imgf.data_ptr(), cls, ep, y_ref.data_ptr(), ws.data_ptr(), s)
    y = torch.full((N, Oc, Lc), 7, dtype=ydt, device=DEV)
    torch.cuda.synchronize()
    L.call("atx_lut_gemm_noalloc", xt.data_ptr(), Rpad, wt.data_ptr(), Opad, N, K, Lc, Oc,
           img16.data_ptr(), imgf.data_ptr(), cls, ep, y.data_ptr(), s)
    torch.cuda.synchronize()
    return y, y_ref, wsb


# (N, K, L, O): stream-K plan (256-KiB slots, forced), then a smaller split-K
# plan, then a smaller whole-tile plan (no scratch)
CALLS = [(64, 256, 3136, 128), (8, 576, 1024, 64), (2, 4, 100, 20)]


@pytest.mark.gpu
@pytest.mark.parametrize("out_kind", [1, 2])          # ATX_OUT_I32, ATX_OUT_DEQUANT
def test_noalloc_matches_workspace_entry_point_on_consecutive_calls(out_kind, monkeypatch):
    """The first call forces the stream-K schedule (ATX_LUT_SCHEDULE, read by
    both entry points); the others take the automatic plan."""
    kinds = []
    for i, (N, K, Lc, Oc) in enumerate(CALLS):
        if i == 0:
            monkeypatch.setenv("ATX_LUT_SCHEDULE", "stream_k")
        else:
            monkeypatch.delenv("ATX_LUT_SCHEDULE", raising=False)
        print(f"noalloc call {i}: N={N} K={K} L={Lc} O={Oc} out_kind={out_kind}", flush=True)
        y, y_ref, wsb = _run(N, K, Lc, Oc, 100 + i, out_kind)
        kinds.append(wsb)
        assert torch.equal(y, y_ref), (N, K, Lc, Oc)
    assert kinds[0] == 255 * 2048 * 32 * 4           # stream-K slots
    assert 0 < kinds[1] < kinds[0] and kinds[2] == 0


@pytest.mark.gpu
def test_noalloc_repeated_call_clears_stale_slots(monkeypatch):
    """The array keeps the previous call's contents; stream-K slots must be
    cleared by every call (the same problem twice gives the same sums)."""
    monkeypatch.setenv("ATX_LUT_SCHEDULE", "stream_k")
    N, K, Lc, Oc = CALLS[0]
    y1, y_ref, _ = _run(N, K, Lc, Oc, 7, L.ATX_OUT_I32)
    y2, _, _ = _run(N, K, Lc, Oc, 7, L.ATX_OUT_I32)
    assert torch.equal(y1, y_ref) and torch.equal(y2, y_ref)


def test_noalloc_rejects_oversized_forced_split_on_the_host():
    """K > 32768 forces two int32 partial slices; with R*O*4*2 > 64 MiB the
    entry point returns ATX_ERANGE before any device call (runs on the CPU:
    the pointers are never dereferenced)."""
    lib = L.load()
    N, K, Lc, Oc = 1, 40000, 65536, 256
    Rpad = L.round_up(N * Lc, L.ROW_TILE)
    ep = L.GemmEpilogue(L.ATX_OUT_I32, None, None, None)
    dummy = ctypes.c_void_p(256)
    rc = lib.atx_lut_gemm_noalloc(dummy, Rpad, dummy, Oc, N, K, Lc, Oc, dummy, dummy,
                                  L.ATX_LUT_U16, ep, dummy, None)
    assert rc == -3
    assert b"scratch" in lib.atx_last_error()
