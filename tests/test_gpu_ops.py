"""GPU parity of every HIP entry point against the CPU oracle (seeded inputs).

Bar: integer / index results bit-exact (int64 oracle); fp32 results of the
fake-quant, EMA and qparam kernels bit-exact (they restate torch's op
sequence); gradients within rel 1e-5 / abs 1e-4 (fp32 accumulation order).
"""
import zlib

import numpy as np
import pytest
import torch

from approxtorch_amd.backend import _lib as LB
from approxtorch_amd.backend import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-5, 1e-4


def gen(seed):
    return np.random.default_rng(seed)


def t(a, dtype=None):
    return torch.as_tensor(np.ascontiguousarray(a), device=DEV, dtype=dtype)


def luts(seed):
    r = gen(seed)
    v = np.arange(256)
    a = v - 128
    return {
        "asym": (37 * v[:, None] - 19 * v[None, :] + 11).reshape(-1),       # int16
        "exact_int8": (a[:, None] * a[None, :]).reshape(-1),                 # int16
        "trunc4": (((a[:, None] * a[None, :]) >> 4) << 4).reshape(-1),       # config 2
        "u16_c5": ((v[:, None] * v[None, :]) & ~63).reshape(-1),            # config 5 (uint16)
        "i16_edge": np.clip(r.integers(-40000, 40000, 65536), -32767, 32767),
        "perturbed": np.clip((a[:, None] * a[None, :]) +
                             np.rint(r.normal(0, 1, (256, 256)) *
                                     (0.02 * np.abs(a[:, None] * a[None, :]) + 1)),
                             -32768, 32767).reshape(-1),
    }


SHAPES = [(1, 1, 1, 1), (2, 5, 7, 3), (3, 33, 9, 17), (2, 576, 64, 64), (1, 300, 1100, 65),
          (4, 64, 49, 130), (1, 4608, 49, 64), (2, 3, 1024, 64), (8, 576, 1024, 64)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("lut_name", ["asym", "perturbed"])
def test_bgemm_int8_u8_input_bit_exact(shape, lut_name):
    N, K, L, Oc = shape
    r = gen(zlib.crc32(repr((shape, lut_name)).encode()))
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wv = r.integers(-128, 128, (Oc, K)).astype(np.float32)
    lut = luts(7)[lut_name]
    xg = t(xi)
    y, xq, wq = ops.bgemm_fake_int8_claude_save(xg, t(wv), t(lut, torch.float32))
    assert xq.data_ptr() == xg.data_ptr()          # _save aliases a uint8 x
    want = O.lut_gemm_i64(xi, (wv + 128).astype(np.uint8), lut)
    assert np.array_equal(wq.cpu().numpy(), (wv + 128).astype(np.uint8))
    assert np.array_equal(y.cpu().numpy(), want.astype(np.float32))


NARROW_GEMM_SHAPES = SHAPES + [(1, 2304, 196, 256), (3, 130, 200, 2048), (1, 40, 3136, 300)]


@pytest.mark.parametrize("shape", NARROW_GEMM_SHAPES)
@pytest.mark.parametrize("lut_name", ["perturbed", "u16_c5", "i16_edge"])
@pytest.mark.parametrize("wbase", [0, 120, 240])
def test_lut_gemm_narrow_bit_exact(shape, lut_name, wbase):
    """LUT GEMM of weights with 16 distinct indices on the int8 matrix cores
    (atx_lut_gemm_narrow): exact int32 sums against the int64 oracle for
    int16 and uint16 tables (extreme entries included), row tiles of 256 and
    channel tiles of 128 with tails, K % 4 != 0, L % 4 != 0, and split-K
    plans (few tiles, long K); the fp32 and dequant epilogues equal the
    table-gather kernel's bit for bit."""
    N, K, L, Oc = shape
    r = gen(zlib.crc32(repr(("narrow_gemm", shape, lut_name, wbase)).encode()))
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(wbase, wbase + 16, (Oc, K), dtype=np.uint8)
    lut = t(luts(9)[lut_name], torch.float32)
    xt, Rpad = ops.pack_rows_u8(t(xi))
    _, wt, Opad = ops._pack_w(t(wi), 0)
    want = O.lut_gemm_i64(xi, wi, luts(9)[lut_name])
    y = torch.empty((N, Oc, L), dtype=torch.int32, device=DEV)
    ops._gemm(xt, Rpad, wt, Opad, N, K, L, Oc, lut, ops.L.ATX_OUT_I32, y, wbase=wbase)
    assert np.array_equal(y.cpu().numpy().astype(np.int64), want)
    if lut_name == "u16_c5":
        sx = t(np.array([0.37], np.float32))
        sw = t((r.random(Oc) + 0.5).astype(np.float32))
        bias = t(r.standard_normal(Oc).astype(np.float32))
        for kind, args in ((ops.L.ATX_OUT_F32, ()), (ops.L.ATX_OUT_DEQUANT, (sx, sw, bias))):
            a = torch.empty((N, Oc, L), dtype=torch.float32, device=DEV)
            b = torch.empty_like(a)
            ops._gemm(xt, Rpad, wt, Opad, N, K, L, Oc, lut, kind, a, *args, wbase=wbase)
            ops._gemm(xt, Rpad, wt, Opad, N, K, L, Oc, lut, kind, b, *args)
            assert torch.equal(a, b)


def test_lut_gemm_narrow_beyond_int32_pass():
    """K > 32768 with uint16 entries: the plan splits K into exact int32
    passes and the reduce sums them in int64 (sums above 2^31)."""
    N, K, L, Oc = 1, 40000, 8, 20
    r = gen(57)
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 16, (Oc, K), dtype=np.uint8)
    lut_np = r.integers(60000, 65536, 65536)        # uint16 class, large entries
    xt, Rpad = ops.pack_rows_u8(t(xi))
    _, wt, Opad = ops._pack_w(t(wi), 0)
    want = O.lut_gemm_i64(xi, wi, lut_np)
    assert want.max() > 2 ** 31
    y = torch.empty((N, Oc, L), dtype=torch.float32, device=DEV)
    ops._gemm(xt, Rpad, wt, Opad, N, K, L, Oc, t(lut_np, torch.float32), ops.L.ATX_OUT_F32, y,
              wbase=0)
    assert np.array_equal(y.cpu().numpy(), want.astype(np.float32))


@pytest.mark.parametrize("shape", NARROW_GEMM_SHAPES + [(2, 40000, 8, 20)])
@pytest.mark.parametrize("lut_name", ["u16_c5", "perturbed"])
@pytest.mark.parametrize("with_bias", [True, False])
def test_lut_gemm_narrow_uint8_epilogue(shape, lut_name, with_bias):
    """atx_lut_gemm_narrow_uint8: the uint8 layer's zero-point correction and
    dequant in the matrix-core GEMM's epilogue (and in the split-K reduce:
    the (1, 2304, 196, 256) and K > 32768 shapes split) equal the fp32 GEMM
    followed by atx_uint8_dequant bit for bit, and the oracle's int64 sums
    corrected in fp64 within 1e-6 of the terms' magnitude (five fp32
    roundings)."""
    N, K, L, Oc = shape
    r = gen(zlib.crc32(repr(("narrow_u8", shape, lut_name, with_bias)).encode()))
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 16, (Oc, K), dtype=np.uint8)
    lut_np = luts(9)[lut_name]
    lut = t(lut_np, torch.float32)
    xt, Rpad = ops.pack_rows_u8(t(xi))
    _, wt, Opad = ops._pack_w(t(wi), 0)
    xsum = xi.astype(np.float64).sum(axis=1).astype(np.float32)          # [N, L], exact
    wsum = wi.astype(np.float64).sum(axis=1).astype(np.float32)          # [O], exact
    zx = np.array([r.integers(0, 256)], np.float32)
    zw = r.integers(0, 16, Oc).astype(np.float32)
    sx = np.array([0.0371], np.float32)
    sw = (r.random(Oc) * 0.02 + 0.001).astype(np.float32)
    bias = r.standard_normal(Oc).astype(np.float32) if with_bias else None
    dev = [t(a) for a in (xsum, wsum, zx, zw, sx, sw)]
    tb = None if bias is None else t(bias)
    a = torch.empty((N, Oc, L), dtype=torch.float32, device=DEV)
    ops._gemm(xt, Rpad, wt, Opad, N, K, L, Oc, lut, ops.L.ATX_OUT_F32, a, dev[4], dev[5], tb,
              wbase=0, u8=tuple(dev[:4]))
    b = torch.empty_like(a)
    ops._gemm(xt, Rpad, wt, Opad, N, K, L, Oc, lut, ops.L.ATX_OUT_F32, b, wbase=0)
    ops.uint8_dequant(b, *dev[:4], dev[4], dev[5], tb, K)
    assert torch.equal(a, b)
    S = O.lut_gemm_i64(xi, wi, lut_np).astype(np.float64)
    zo, so = zw.astype(np.float64)[None, :, None], (sx.astype(np.float64) * sw)[None, :, None]
    xs, z = xsum.astype(np.float64)[:, None, :], float(zx[0])
    ws = wsum.astype(np.float64)[None, :, None]
    want = (S - zo * xs - z * ws + K * z * zo) * so
    mag = (np.abs(S) + zo * xs + z * ws + K * z * zo) * so
    if bias is not None:
        want = want + bias.astype(np.float64)[None, :, None]
        mag = mag + np.abs(bias.astype(np.float64))[None, :, None]
    err = np.abs(a.cpu().numpy().astype(np.float64) - want)
    assert (err <= 1e-6 * mag + 1e-30).all(), err.max()


# Stream-K schedule of the LUT GEMM: full rounds of whole tiles, then the
# (tile, 4-table quad) iterations of the remaining tiles dealt out evenly over
# 256 workgroups; a tile cut by a workgroup boundary sums its int32 parts
# atomically into a slot.  Its workspace is 255 slots of 2048 x 32 int32,
# which is how these tests know the schedule was taken.  ATX_LUT_SCHEDULE
# forces it on shapes small enough for the full oracle:
#   (1, 1000, 4096, 40): 4 tiles cut into ~60 segments each, K % 4 != 0,
#                        O % 32 != 0;
#   (2, 2002, 3000, 40): 6 tiles, the last row tile partial, K % 4 != 0;
#   (150, 64, 2048, 64): 300 tiles: one round of 256 whole tiles, then 44
#                        tiles over 256 workgroups (sampled check).
SK_WORKSPACE = 255 * 2048 * 32 * 4
SK_SHAPES = [(1, 1000, 4096, 40), (2, 2002, 3000, 40)]


def _sampled_lut_sums(xi, wi, lut, n, o, l):
    k = np.arange(xi.shape[1])
    idx = xi[n[:, None], k[None, :], l[:, None]].astype(np.int64) * 256 + wi[o][:, :]
    return np.asarray(lut, np.int64)[idx].sum(axis=1)


def _check_sampled(y, xi, wi, lut, r, tiles_o):
    N, K, L = xi.shape
    Oc = wi.shape[0]
    n, o, l = r.integers(0, N, 4096), r.integers(0, Oc, 4096), r.integers(0, L, 4096)
    assert np.array_equal(y[n, o, l].astype(np.int64), _sampled_lut_sums(xi, wi, lut, n, o, l))
    R = N * L
    for tile in range(-(-R // 2048) * tiles_o):    # first / last row and channel of every tile
        tr, to = divmod(tile, tiles_o)
        for rr in (tr * 2048, min(R, tr * 2048 + 2048) - 1):
            nn, ll = divmod(rr, L)
            oo = np.array([to * 32, min(Oc, to * 32 + 32) - 1])
            want = _sampled_lut_sums(xi, wi, lut, np.array([nn, nn]), oo, np.array([ll, ll]))
            assert np.array_equal(y[nn, oo, ll].astype(np.int64), want), (tile, rr)


@pytest.mark.parametrize("shape", SK_SHAPES)
@pytest.mark.parametrize("lut_name", ["perturbed", "u16_c5"])
def test_lut_gemm_stream_k_exact(shape, lut_name, monkeypatch):
    monkeypatch.setenv("ATX_LUT_SCHEDULE", "stream_k")
    N, K, L, Oc = shape
    assert ops.L.query("atx_lut_gemm_workspace_bytes", N, K, L, Oc) == SK_WORKSPACE
    r = gen(zlib.crc32(repr((shape, lut_name)).encode()))
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = luts(5)[lut_name]
    want = O.lut_gemm_i64(xi, wi, lut)
    for _ in range(2):                       # the slots are cleared on every call
        y = ops.lut_gemm_i32(t(xi), t(wi), t(lut, torch.float32))
        assert np.array_equal(y.cpu().numpy().astype(np.int64), want)
    if lut_name == "perturbed":              # fp32 epilogue of the finished tiles
        wv = wi.astype(np.float32) - 128
        yf = ops.bgemm_fake_int8_claude(t(xi), t(wv), t(lut, torch.float32))
        assert np.array_equal(yf.cpu().numpy(), want.astype(np.float32))
    monkeypatch.setenv("ATX_LUT_SCHEDULE", "split")
    assert ops.L.query("atx_lut_gemm_workspace_bytes", N, K, L, Oc) != SK_WORKSPACE
    y = ops.lut_gemm_i32(t(xi), t(wi), t(lut, torch.float32))
    assert np.array_equal(y.cpu().numpy().astype(np.int64), want)


def test_lut_gemm_stream_k_full_round_then_tail_sampled(monkeypatch):
    monkeypatch.setenv("ATX_LUT_SCHEDULE", "stream_k")
    N, K, L, Oc = 150, 64, 2048, 64
    assert ops.L.query("atx_lut_gemm_workspace_bytes", N, K, L, Oc) == SK_WORKSPACE
    r = gen(23)
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = luts(6)["i16_edge"]
    y = ops.lut_gemm_i32(t(xi), t(wi), t(lut, torch.float32)).cpu().numpy()
    _check_sampled(y, xi, wi, lut, r, 2)


def test_lut_gemm_resnet_layer_plans_sampled(monkeypatch):
    """ResNet-50 layer2 1x1 conv at batch 64 (R = 200704, K = 256, O = 128,
    392 tiles): the cost model picks stream-K; the split-K-only plan (rows
    per tile and split count from the model) gives the same exact sums
    (sampled)."""
    N, K, L, Oc = 64, 256, 3136, 128
    r = gen(29)
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = luts(8)["perturbed"]
    for sched in ("auto", "split"):
        monkeypatch.setenv("ATX_LUT_SCHEDULE", sched)
        ws = ops.L.query("atx_lut_gemm_workspace_bytes", N, K, L, Oc)
        assert (ws == SK_WORKSPACE) == (sched == "auto")
        y = ops.lut_gemm_i32(t(xi), t(wi), t(lut, torch.float32)).cpu().numpy()
        _check_sampled(y, xi, wi, lut, r, 4)


@pytest.mark.parametrize("rows", [768, 1280, 1536, 1792])
@pytest.mark.parametrize("splits", [1, 3])
def test_lut_gemm_row_tiles_exact(rows, splits, monkeypatch):
    """Tiles of fewer than 2048 rows (whole waves; the waves past the tile
    only build tables) with and without split-K: exact against the oracle.
    R = 3300 rows: 768 -> 5 tiles, 1280 -> 3, 1792 -> 2 (the last partial);
    1536 would need 4608 padded rows and falls back to the default tile."""
    monkeypatch.setenv("ATX_LUT_ROWS", str(rows))
    monkeypatch.setenv("ATX_LUT_SPLITS", str(splits))
    N, K, L, Oc = 3, 300, 1100, 70
    r = gen(zlib.crc32(repr(("rows", rows, splits)).encode()))
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = luts(4)["i16_edge"]
    y = ops.lut_gemm_i32(t(xi), t(wi), t(lut, torch.float32))
    assert np.array_equal(y.cpu().numpy().astype(np.int64), O.lut_gemm_i64(xi, wi, lut))


def test_lut_gemm_config3_full_shape_sampled():
    """Config 3 at its headline shape: B=32 x [4096 x 2304] int8 by [2304 x 256],
    perturbed LUT.  The int32 sums (exact) and the fp32 output of the
    reference op (bgemm_fake_int8_forward_cuda_claude, the bench path) are
    checked on 4096 random outputs plus the corners of every tile."""
    N, K, L, Oc = 32, 2304, 4096, 256
    r = gen(33)
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = luts(3)["perturbed"]
    xg, lg = t(xi), t(lut, torch.float32)
    y = ops.lut_gemm_i32(xg, t(wi), lg).cpu().numpy()
    _check_sampled(y, xi, wi, lut, r, Oc // 32)
    del y
    yf = ops.bgemm_fake_int8_claude(xg, t(wi.astype(np.float32) - 128), lg).cpu().numpy()
    n, o, l = r.integers(0, N, 4096), r.integers(0, Oc, 4096), r.integers(0, L, 4096)
    want = _sampled_lut_sums(xi, wi, lut, n, o, l).astype(np.float32)   # correctly rounded
    assert np.array_equal(yf[n, o, l], want)


@pytest.mark.parametrize("lut_name", ["asym", "exact_int8", "trunc4", "u16_c5", "i16_edge"])
def test_lut_gemm_int32_exact_all_integer_classes(lut_name):
    r = gen(11)
    N, K, L, Oc = 3, 700, 333, 70
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = luts(3)[lut_name]
    y = ops.lut_gemm_i32(t(xi), t(wi), t(lut, torch.float32))
    assert np.array_equal(y.cpu().numpy().astype(np.int64), O.lut_gemm_i64(xi, wi, lut))


def test_bgemm_float_inputs_quantize_like_reference():
    # fp32 x, w holding quantized values (plus half-integers and out-of-range
    # values: index = clamp(rint(v) + 128, 0, 255))
    r = gen(5)
    x = r.integers(-140, 140, (2, 50, 40)).astype(np.float32)
    x[0, 0, :6] = [0.5, 1.5, -0.5, -2.5, 127.5, np.nan]
    w = r.integers(-128, 128, (9, 50)).astype(np.float32)
    lut = luts(1)["asym"]
    y, xq, wq = ops.bgemm_fake_int8_claude_save(t(x), t(w), t(lut, torch.float32))
    xi = O.quant_index(x, 128)
    assert np.array_equal(xq.cpu().numpy(), xi)
    assert np.array_equal(y.cpu().numpy(),
                          O.lut_gemm_i64(xi, O.quant_index(w, 128), lut).astype(np.float32))


def test_int8_equals_uint8_shifted():
    r = gen(9)
    x = r.integers(-128, 128, (3, 64, 50)).astype(np.float32)
    w = r.integers(-128, 128, (20, 64)).astype(np.float32)
    lut = t(luts(2)["perturbed"], torch.float32)
    a = ops.bgemm_fake_int8_claude(t(x), t(w), lut)
    b = ops.bgemm_fake_uint8_claude(t(x + 128), t(w + 128), lut)
    assert torch.equal(a, b)


def test_fp32_lut_fallback_matches_sequential_fp32():
    r = gen(4)
    xi = r.integers(0, 256, (2, 100, 37), dtype=np.uint8)
    w = r.integers(-128, 128, (11, 100)).astype(np.float32)
    lut = (r.integers(-4000, 4000, 65536) / 2 + 0.25).astype(np.float32)   # non-integer
    y = ops.bgemm_fake_int8_claude(t(xi), t(w), t(lut))
    want = O.lut_gemm_f32(xi, (w + 128).astype(np.uint8), lut)
    assert np.array_equal(y.cpu().numpy(), want)          # same ascending-k fp32 order


F32_SHAPES = [(2, 100, 37, 11), (3, 9, 64, 40), (1, 257, 4100, 33), (2, 4, 100, 16),
              (1, 3, 2051, 17), (2, 0, 10, 5)]


@pytest.mark.parametrize("shape", F32_SHAPES)
def test_fp32_lut_tiled_kernel(shape):
    """The tiled fp32-class path (LDS tables from the fp32 image, ascending
    k) equals the sequential fp32 sum bit for bit, through row tiles, ragged
    channel tiles, K not a multiple of 4, L % 4 != 0 and K = 0, and its
    dequant epilogue rounds like sx * sw[o] * y + bias in fp32."""
    N, K, Lc, Oc = shape
    r = gen(40 + K)
    xi = r.integers(0, 256, (N, K, Lc), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = (r.standard_normal(65536) * 1000).astype(np.float32)
    want = O.lut_gemm_f32(xi, wi, lut)
    Rpad = LB.round_up(max(N * Lc, 1), LB.ROW_TILE)
    xt = torch.zeros((max(LB.operand_rows(K), 1), Rpad), dtype=torch.int16, device=DEV)
    xg = t(xi)
    if K:
        LB.call("atx_pack_x_u8", LB.ptr(xg), N, K, Lc, LB.ptr(xt), Rpad, None, LB.stream_of(xg))
    _, wt, Opad = ops._pack_w(t(wi), 0)
    lt = t(lut)
    y = torch.full((N, Oc, Lc), float("nan"), device=DEV)
    ops._gemm(xt, Rpad, wt, Opad, N, K, Lc, Oc, lt, LB.ATX_OUT_F32, y)
    assert np.array_equal(y.cpu().numpy(), want)
    sx = np.float32([0.37])
    sw = (r.random(Oc) + 0.5).astype(np.float32)
    bias = r.standard_normal(Oc).astype(np.float32)
    y2 = torch.full((N, Oc, Lc), float("nan"), device=DEV)
    ops._gemm(xt, Rpad, wt, Opad, N, K, Lc, Oc, lt, LB.ATX_OUT_DEQUANT, y2, t(sx), t(sw), t(bias))
    want2 = want * (sx[0] * sw)[None, :, None] + bias[None, :, None]
    assert np.array_equal(y2.cpu().numpy(), want2.astype(np.float32))


def test_lut_cache_tracks_in_place_updates():
    r = gen(6)
    xi = t(r.integers(0, 256, (1, 8, 8), dtype=np.uint8))
    w = t(r.integers(-128, 128, (4, 8)).astype(np.float32))
    lut = t(luts(0)["asym"], torch.float32)
    y0 = ops.bgemm_fake_int8_claude(xi, w, lut)
    lut.mul_(2)                                            # bumps the version counter
    y1 = ops.bgemm_fake_int8_claude(xi, w, lut)
    assert torch.equal(y1, 2 * y0)


def test_empty_and_degenerate_shapes():
    lut = t(luts(0)["asym"], torch.float32)
    y = ops.bgemm_fake_int8_claude(torch.zeros(2, 0, 5, device=DEV),
                                   torch.zeros(3, 0, device=DEV), lut)
    assert y.shape == (2, 3, 5) and torch.count_nonzero(y) == 0
    y = ops.bgemm_fake_int8_claude(torch.zeros(0, 4, 5, device=DEV),
                                   torch.zeros(3, 4, device=DEV), lut)
    assert y.shape == (0, 3, 5)
    with pytest.raises(RuntimeError, match="x.size"):
        ops.bgemm_fake_int8_claude(torch.zeros(1, 4, 5, device=DEV),
                                   torch.zeros(3, 5, device=DEV), lut)
    with pytest.raises(RuntimeError, match="float32"):
        ops.bgemm_fake_int8_claude(torch.zeros(1, 4, 5, device=DEV),
                                   torch.zeros(3, 4, device=DEV), lut.int())


GEOMS = [((3, 3), (1, 1), (1, 1), (1, 1)), ((7, 7), (2, 2), (3, 3), (1, 1)),
         ((1, 1), (2, 2), (0, 0), (1, 1)), ((3, 3), (1, 2), (2, 0), (2, 1)),
         ((3, 3), (2, 2), (1, 1), (1, 1))]


@pytest.mark.parametrize("geom", GEOMS)
@pytest.mark.parametrize("dtype", ["int8", "uint8", "float32"])
def test_im2col_u8(geom, dtype):
    k, s, p, d = geom
    r = gen(8)
    if dtype == "int8":
        img = r.integers(-128, 128, (2, 3, 13, 11)).astype(np.int8)
    elif dtype == "uint8":
        img = r.integers(0, 256, (2, 3, 13, 11)).astype(np.uint8)
    else:
        img = r.integers(-130, 130, (2, 3, 13, 11)).astype(np.float32)
    got = ops.im2col_u8(t(img), k, s, p, d).cpu().numpy()
    assert np.array_equal(got, O.im2col_index(O.image_index(img, 128), k, s, p, d, 128))


@pytest.mark.parametrize("geom", GEOMS)
def test_lut_conv_forward_matches_oracle(geom):
    k, s, p, d = geom
    r = gen(12)
    img = r.integers(-127, 128, (3, 8, 15, 14)).astype(np.float32)
    w = r.integers(-127, 128, (70, 8 * k[0] * k[1])).astype(np.float32)
    lut = luts(4)["perturbed"]
    g = ops.conv_geom(img.shape, k, s, p, d)
    y, wq = ops.conv_forward(t(img), t(w), t(lut, torch.float32), g, 128, 128)
    xi = O.im2col_index(O.image_index(img, 128), k, s, p, d, 128)
    want = O.lut_gemm_i64(xi, (w + 128).astype(np.uint8), lut)
    assert np.array_equal(y.cpu().numpy(), want.astype(np.float32))


# (N, C, H, W, geometry): K = C*KH*KW of 8 or 27 runs in one pass; 72, 392
# and 1152 run split-K (int32 partials + reduce); L = 256 and 64 store
# four-row vectors, the others row by row.
DEQ_CASES = [(3, 8, 15, 14, GEOMS[0]), (2, 8, 16, 16, GEOMS[0]), (2, 8, 16, 16, GEOMS[2]),
             (2, 8, 17, 17, GEOMS[1]), (4, 3, 16, 16, GEOMS[0]), (1, 128, 8, 8, GEOMS[0])]


@pytest.mark.parametrize("case", DEQ_CASES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_fused_dequant_and_int32_epilogues(case, with_bias):
    N, C, H, W, (k, s, p, d) = case
    r = gen(zlib.crc32(repr((case, with_bias)).encode()))
    img = r.integers(-127, 128, (N, C, H, W)).astype(np.float32)
    Oc = 70
    w = r.integers(-127, 128, (Oc, C * k[0] * k[1])).astype(np.float32)
    lut = luts(4)["perturbed"]
    g = ops.conv_geom(img.shape, k, s, p, d)
    xi = O.im2col_index(O.image_index(img, 128), k, s, p, d, 128)
    want_i = O.lut_gemm_i64(xi, (w + 128).astype(np.uint8), lut)
    sx = np.array([0.0173], np.float32)
    sw = r.uniform(1e-3, 5e-2, Oc).astype(np.float32)
    bias = r.standard_normal(Oc).astype(np.float32) if with_bias else None
    y, _ = ops.conv_forward(t(img), t(w), t(lut, torch.float32), g, 128, 128,
                            out_kind=ops.L.ATX_OUT_DEQUANT, sx=t(sx), sw=t(sw),
                            bias=None if bias is None else t(bias))
    # the epilogue's fp32 sequence: sc = sx * sw[o]; t = float(v) * sc; bias + t
    sc = (sx[0] * sw)[None, :, None]
    want = want_i.astype(np.float32) * sc
    if bias is not None:
        want = bias[None, :, None] + want
    assert np.array_equal(y.cpu().numpy(), want)
    yi, _ = ops.conv_forward(t(img), t(w), t(lut, torch.float32), g, 128, 128,
                             out_kind=ops.L.ATX_OUT_I32)
    assert yi.dtype == torch.int32
    assert np.array_equal(yi.cpu().numpy().astype(np.int64), want_i)


def test_lut_map_and_pad():
    r = gen(13)
    table = r.standard_normal(256).astype(np.float32)
    for arr in (r.integers(-128, 128, (2, 3, 5, 4)).astype(np.int8),
                r.integers(0, 256, (2, 3, 5, 4)).astype(np.uint8),
                r.integers(-130, 130, (2, 3, 5, 4)).astype(np.float32)):
        idx = O.image_index(arr, 128)
        assert np.array_equal(ops.lut_map(t(arr), t(table)).cpu().numpy(), O.lut_map(idx, table))
        assert np.array_equal(ops.lut_map_pad(t(arr), t(table), (2, 1)).cpu().numpy(),
                              O.lut_map_pad(idx, table, (2, 1)))


# ---------------------------------------------------------------- fake-quant
def special_x(seed, n=20000):
    r = gen(seed)
    x = (r.standard_normal(n) * 3).astype(np.float32)
    x[:12] = [0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 127.5, -127.5, 300, -300, np.nan, -0.0]
    return x


@pytest.mark.parametrize("scale", [0.023, 1.0, 0.0, 1e-30])
def test_fakequant_symmetric_bitwise(scale):
    x = special_x(1)
    s = np.float32(scale)
    q, m, _ = ops.fakequant_per_tensor(t(x), t(np.array([s])), -127, 127)
    qo, mo = O.fakequant(x, s, -127, 127)
    assert np.array_equal(q.cpu().numpy(), qo, equal_nan=True)
    assert np.array_equal(m.cpu().numpy(), mo)
    go = gen(2).standard_normal(x.size).astype(np.float32)
    gx = ops.fakequant_per_tensor_backward(t(go), m, t(np.array([s])))
    assert np.array_equal(gx.cpu().numpy(), O.fakequant_backward(go, mo, s))


def decode_operand(xt, K, R):
    """LUT indices [K, R] of a row-offset operand xt [Kpad][Rpad]: slot s of
    row r holds tap (s & ~3) | ((r//4 + s) & 3) as v*256 + ((v >> 1) & 3)*16;
    asserts the padding entries are 0."""
    xt = xt.astype(np.int64) & 0xFFFF
    Kp, Rp = xt.shape
    s = np.arange(Kp)[:, None]
    r = np.arange(Rp)[None, :]
    tap = (s & ~3) | (((r >> 2) + s) & 3)
    v = xt >> 8
    assert np.array_equal(xt, np.where((tap < K) & (r < R), v * 256 + ((v >> 1) & 3) * 16, 0))
    out = np.zeros((K, R), np.int64)
    keep = (tap < K) & (r < R)
    out[tap[keep], np.broadcast_to(r, tap.shape)[keep]] = v[keep]
    return out


# Implicit-im2col operand at sizes whose grids take slot runs of 32, 16 and
# 8 (the launch shortens the run until it has 2048 blocks; the small conv
# tests above take runs of 4): (N, C, H, W, padding).
IM_RUN_CASES = [(2, 256, 128, 128, 1), (2, 128, 128, 128, 1), (1, 512, 64, 64, 0)]


@pytest.mark.parametrize("case", IM_RUN_CASES)
def test_im2col_rows_slot_runs_sampled(case):
    N, C, H, W, p = case
    r = gen(zlib.crc32(repr(case).encode()))
    img = r.integers(-128, 128, (N, C, H, W)).astype(np.int8)
    g = ops.conv_geom(img.shape, (3, 3), (1, 1), (p, p), (1, 1))
    _, _, (xt, Rpad) = ops.conv_forward(t(img), torch.zeros(1, C * 9, device=DEV),
                                        t(np.zeros(65536, np.float32)), g, 128, 128,
                                        return_operand=True)
    K, OH, OW = C * 9, g.OH, g.OW
    R = N * OH * OW
    # sampled (slot, row) pairs plus every row of the first and last slots
    slot = np.concatenate([r.integers(0, K, 30000), np.zeros(R, np.int64),
                           np.full(R, K - 1)])
    row = np.concatenate([r.integers(0, Rpad, 30000), np.arange(R), np.arange(R)])
    got = xt[t(slot), t(row)].cpu().numpy().astype(np.int64) & 0xFFFF
    k = (slot & ~3) | (((row >> 2) + slot) & 3)
    live = (k < K) & (row < R)
    c, kh, kw = k // 9, (k % 9) // 3, k % 3
    n, rem = row // (OH * OW), row % (OH * OW)
    ih, iw = rem // OW - p + kh, rem % OW - p + kw
    inside = live & (ih >= 0) & (ih < H) & (iw >= 0) & (iw < W)
    v = np.full(slot.shape, 128, np.int64)       # padding taps read index 128
    v[inside] = img[n[inside], c[inside], ih[inside], iw[inside]].astype(np.int64) + 128
    want = np.where(live, v * 256 + ((v >> 1) & 3) * 16, 0)
    assert np.array_equal(got, want)


# (N, C, H, W): L = 49 and K = 6 take the element-wise path, L = 64 / 784
# the 16-byte one; K = 40 and 64 span two slot runs; the last is a 1x1 pixel.
# With L % 4 == 0 the byte image's im2col reads 4-byte row quads; (3, 6, 4, 4)
# has K % 4 != 0 and padding rows past N*L.
FQ_ROWS_CASES = [(2, 6, 7, 7), (3, 40, 8, 8), (2, 64, 28, 28), (5, 3, 1, 1), (3, 6, 4, 4)]


@pytest.mark.parametrize("shape", FQ_ROWS_CASES)
@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("misalign", [False, True])
def test_fakequant_rows_matches_fakequant_then_im2col(shape, signed, misalign):
    N, C, H, W = shape
    n = N * C * H * W
    x = special_x(zlib.crc32(repr(shape).encode()), max(n, 12))[:n]
    base = torch.zeros(n + 1, device=DEV)
    base[int(misalign):int(misalign) + n] = t(x)
    xd = base[int(misalign):int(misalign) + n].view(N, C, H, W)
    s = np.float32(0.023)
    if signed:
        qmin, qmax, off, z, zt = -128, 127, 128, None, None
    else:
        qmin, qmax, off = 0, 255, 0
        z = np.float32(113)
        zt = t(np.array([z]))
    mask, (xt, Rpad) = ops.fakequant_rows(xd, t(np.array([s])), qmin, qmax, off,
                                          zero_point=zt)
    qo, mo = O.fakequant(x, s, qmin, qmax, zero=z)
    assert np.array_equal(mask.cpu().numpy().reshape(-1), mo)
    idx = O.quant_index(qo, off).reshape(N, C, H * W)
    want = idx.transpose(1, 0, 2).reshape(C, N * H * W)
    assert np.array_equal(decode_operand(xt.cpu().numpy(), C, N * H * W), want)
    # bit-identical to the byte image through the conv's im2col
    _, m2, q8 = ops.fakequant_per_tensor(xd, t(np.array([s])), qmin, qmax, zero_point=zt,
                                         want_q=False,
                                         q8_dtype=torch.int8 if signed else torch.uint8)
    g = ops.conv_geom((N, C, H, W), (1, 1), (1, 1), (0, 0), (1, 1))
    _, _, (xt2, Rpad2) = ops.conv_forward(q8, torch.zeros(1, C, device=DEV),
                                          t(np.zeros(65536, np.float32)), g, off, off,
                                          return_operand=True)
    assert Rpad == Rpad2 and torch.equal(xt, xt2) and torch.equal(mask, m2)


def test_fakequant_rows_empty_batch_writes_only_padding():
    x = torch.zeros(0, 6, 7, 7, device=DEV)
    mask, (xt, Rpad) = ops.fakequant_rows(x, t(np.array([np.float32(0.5)])), -128, 127, 128)
    assert mask.shape == x.shape and Rpad == 2048 and tuple(xt.shape) == (8, 2048)
    assert int(xt.abs().sum()) == 0


def test_fakequant_asymmetric_and_per_channel_bitwise():
    x = special_x(3).reshape(20, 1000)
    s, z = np.float32(0.031), np.float32(113)
    q, m, _ = ops.fakequant_per_tensor(t(x), t(np.array([s])), 0, 255, zero_point=t(np.array([z])))
    qo, mo = O.fakequant(x, s, 0, 255, zero=z)
    assert np.array_equal(q.cpu().numpy(), qo, equal_nan=True)
    assert np.array_equal(m.cpu().numpy(), mo)
    sc = gen(4).random(20).astype(np.float32) * 0.05
    sc[3] = 0
    q, m, wq, wt, Opad = ops.fakequant_per_channel(t(x), t(sc), -15, 15, offset=128, want_wt=True)
    qo, mo = O.fakequant(x, sc.reshape(20, 1), -15, 15)
    assert np.array_equal(q.cpu().numpy(), qo, equal_nan=True)
    assert np.array_equal(m.cpu().numpy(), mo)
    idx = O.quant_index(qo, 128)
    assert np.array_equal(wq.cpu().numpy(), idx)
    assert np.array_equal(wt.cpu().numpy()[:, :20], idx.T)


@pytest.mark.parametrize("m", [0.05, 0.1])
def test_ema_kernels_bitwise(m):
    from approxtorch_amd.backend import _lib as L
    from approxtorch_amd.nn.Conv2d_int8 import _ema_coeffs
    r = gen(21)
    x = (r.standard_normal(300001) * 2.5).astype(np.float32)
    xg = t(x)
    scale = t(np.array([0.0371], dtype=np.float32))
    stat = torch.empty((), device=DEV)
    ws = ops._reduce_ws(xg.device)
    st = L.stream_of(xg)
    m32, om32 = _ema_coeffs(m)
    L.call("atx_absmax", xg.data_ptr(), x.size, ws.data_ptr(), stat.data_ptr(), st)
    L.call("atx_ema_absmax_apply", stat.data_ptr(), 127.0, m32, om32, scale.data_ptr(), st)
    assert scale.item() == O.ema_absmax(x, np.float32(0.0371), m)
    # the fused reduction + EMA (single-process layers) gives the same bits
    scale2 = t(np.array([0.0371], dtype=np.float32))
    stat2 = torch.empty((), device=DEV)
    L.call("atx_absmax_ema", xg.data_ptr(), x.size, ws.data_ptr(), stat2.data_ptr(), 127.0,
           m32, om32, scale2.data_ptr(), st)
    assert stat2.item() == stat.item() and scale2.item() == scale.item()
    w = (r.standard_normal((33, 3, 3, 3)) * 0.1).astype(np.float32)
    w[5] = 0
    sw = (r.random(33) * 0.01).astype(np.float32)
    swg = t(sw.copy())
    wg = t(w)
    L.call("atx_weight_scale_ema", wg.data_ptr(), 33, 27, 7.0, m32, om32, 0, swg.data_ptr(), st)
    assert np.array_equal(swg.cpu().numpy(), O.weight_scale_ema(w, sw, m, 7))
    L.call("atx_weight_scale_ema", wg.data_ptr(), 33, 27, 7.0, 1.0, 0.0, 1, swg.data_ptr(), st)
    assert np.array_equal(swg.cpu().numpy(), O.weight_scale_reset(w, 7))
    # uint8 activation min/max EMA + qparams
    mn, mx = torch.empty((), device=DEV), torch.empty((), device=DEV)
    bufs = [t(np.array([v], dtype=np.float32)) for v in (-0.2, 1.7, 0.0, 0.0)]
    L.call("atx_minmax", xg.data_ptr(), x.size, ws.data_ptr(), mn.data_ptr(), mx.data_ptr(), st)
    L.call("atx_ema_minmax_apply", mn.data_ptr(), mx.data_ptr(), m32, om32, 255,
           *[b.data_ptr() for b in bufs], st)
    want = O.ema_minmax(x, np.float32(-0.2), np.float32(1.7), m)
    assert [b.item() for b in bufs] == [float(v) for v in want]
    bufs2 = [t(np.array([v], dtype=np.float32)) for v in (-0.2, 1.7, 0.0, 0.0)]
    mn2, mx2 = torch.empty((), device=DEV), torch.empty((), device=DEV)
    L.call("atx_minmax_ema", xg.data_ptr(), x.size, ws.data_ptr(), mn2.data_ptr(),
           mx2.data_ptr(), m32, om32, 255, *[b.data_ptr() for b in bufs2], st)
    assert (mn2.item(), mx2.item()) == (mn.item(), mx.item())
    assert [b.item() for b in bufs2] == [float(v) for v in want]
    # uint8 weights
    wmin, wmax = (r.standard_normal(33) * 0.1).astype(np.float32), \
        (r.random(33) * 0.1).astype(np.float32)
    g4 = [t(wmin.copy()), t(wmax.copy()), torch.empty(33, device=DEV), torch.empty(33, device=DEV)]
    L.call("atx_weight_minmax_ema", wg.data_ptr(), 33, 27, m32, om32, 15,
           *[b.data_ptr() for b in g4], st)
    want = O.weight_minmax_ema(w, wmin, wmax, m, 15)
    for got, exp in zip(g4, want):
        assert np.array_equal(got.cpu().numpy(), exp)


def test_torch_gpu_divides_by_numbers_via_the_reciprocal():
    """The reference's scale statements run by torch on this GPU -- abs_max /
    ((qmax - qmin) / 2), absmax / qmax_w, (mx - mn) / qmax with python-number
    divisors (nn/Conv2d_int8.py:144,155,166; nn/Conv2d_uint8.py:21) -- equal
    the oracle's v * fp32(1 / number) bit for bit, where exact division would
    differ: the device semantics the statistic kernels and the oracle follow."""
    r = gen(23)
    v = (r.random(100000) * 50).astype(np.float32)
    vg = t(v)
    for number in (127.0, 7, 255, 15):
        got = (vg / number).cpu().numpy()
        assert np.array_equal(got, O.div_by_number(v, number))
    assert ((vg / 127.0).cpu().numpy() != v / np.float32(127)).sum() > 100
    # the EMA statement itself, on a 0-dim device statistic, for many inputs
    m = 0.05
    old = torch.tensor(0.0371, device=DEV)
    for i in range(200):
        x = (r.standard_normal(257) * (1 + i)).astype(np.float32)
        abs_max = t(x).abs().max()
        want = (m * (abs_max / ((127 - -127) / 2)) + (1 - m) * old).item()
        assert want == O.ema_absmax(x, np.float32(0.0371), m)


# ------------------------------------------------------------ backward ops
def close(a, b, absref=None):
    """rel 1e-5 / abs 1e-4.  With absref (the sum of |terms| of each output),
    the relative part is taken against it: an fp32 sum of n terms in any order
    is within n * 6e-8 * sum|terms| of the exact value, so this is the bound
    the reference's own fp32 accumulation order meets (cancelling sums make a
    relative bound on the result itself meaningless)."""
    a = np.asarray(a, dtype=np.float64)
    ref = np.abs(b) if absref is None else absref
    excess = np.abs(a - b) - (ATOL + RTOL * ref)
    assert excess.max() <= 0, f"max excess {excess.max():.3g} at {np.unravel_index(excess.argmax(), a.shape)}"


@pytest.mark.parametrize("xdtype", ["uint8", "int8", "float32"])
def test_bgemm_lre_backward(xdtype):
    r = gen(31)
    N, K, L, Oc = 3, 90, 77, 40
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    q = np.arange(256, dtype=np.float32) - 128
    dx = (0.0003 * q * q - 0.07 * q + 1.25).astype(np.float32)      # test_bgemm_lre_naive.py:55-57
    dw = (2.5 * np.sin(0.031 * q) + 0.004 * q).astype(np.float32)
    go = r.standard_normal((N, Oc, L)).astype(np.float32)
    if xdtype == "uint8":
        xa, wa = xi, wi
    elif xdtype == "int8":
        xa, wa = (xi.astype(np.int16) - 128).astype(np.int8), (wi.astype(np.int16) - 128).astype(np.int8)
    else:
        xa, wa = xi.astype(np.float32) - 128, wi.astype(np.float32) - 128
    gx, gw = ops.bgemm_lre_backward_claude(t(go), t(xa), t(np.ascontiguousarray(wa.T)), t(dx), t(dw))
    ex, ew = O.gemm_grads(go, xi, wi, "lre", (dx, dw))
    close(gx.cpu().numpy(), ex)
    close(gw.cpu().numpy(), ew.T)


@pytest.mark.parametrize("signed", [False, True])
def test_custom_grad_kernels(signed):
    r = gen(41)
    N, K, L, Oc = 2, 45, 130, 70
    xi = r.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    rr, cc = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
    dxl = (rr * 1009 + cc * 7 + (rr * cc) % 31).astype(np.float32) / 1000.0   # test_conv_custom_grad.py:41-44
    dwl = dxl.T.copy()
    go = r.standard_normal((N, Oc, L)).astype(np.float32)
    if signed:
        X, W = (xi.astype(np.int16) - 128).astype(np.int8), (wi.astype(np.int16) - 128).astype(np.int8)
        fdx, fdw = ops.bgemm_custom_grad_int8_dx, ops.bgemm_custom_grad_int8_dw
    else:
        X, W = xi, wi
        fdx, fdw = ops.bgemm_custom_grad_uint8_dx, ops.bgemm_custom_grad_uint8_dw
    gx = fdx(t(X), t(W), t(go), t(dxl.reshape(-1)))
    gw = fdw(t(X), t(W), t(go), t(dwl.reshape(-1)))
    ex, ew = O.gemm_grads(go, xi, wi, "custom", (dxl, dwl))
    ax, aw = O.gemm_grads(np.abs(go), xi, wi, "custom", (np.abs(dxl), np.abs(dwl)))
    close(gx.cpu().numpy(), ex, ax)
    close(gw.cpu().numpy(), ew, aw)


TAP_GEOMS = [((2, 5, 9, 7), (3, 3), (1, 1), (1, 1), (1, 1)), ((3, 130, 6, 5), (3, 3), (2, 2), (1, 1), (1, 1)),
             ((2, 64, 7, 7), (1, 1), (1, 1), (0, 0), (1, 1)), ((1, 200, 11, 13), (3, 3), (1, 2), (2, 2), (2, 1)),
             ((4, 3, 16, 16), (7, 7), (2, 2), (3, 3), (1, 1)), ((2, 6, 9, 7), (1, 1), (2, 2), (0, 0), (1, 1)),
             ((2, 4, 8, 10), (3, 3), (2, 2), (1, 1), (1, 1)), ((1, 3, 11, 9), (3, 3), (2, 2), (2, 2), (2, 2)),
             ((2, 5, 10, 9), (3, 2), (2, 2), (0, 1), (1, 3)), ((2, 150, 12, 8), (3, 3), (1, 1), (1, 1), (1, 1)),
             ((3, 80, 14, 14), (1, 1), (1, 1), (0, 0), (1, 1))]


def fold_f32(col, shape, k, s, p, d):
    """F.fold in fp32 with every pixel's taps added in ascending (kh, kw)
    order from +0: the order the col2im kernels document, so their output is
    this bit for bit."""
    N, C, H, W = shape
    OH, OW = O.out_size(H, W, k, s, p, d)
    padded = np.zeros((N, C, H + 2 * p[0] + s[0] + d[0] * k[0], W + 2 * p[1] + s[1] + d[1] * k[1]),
                      dtype=np.float32)
    c6 = np.asarray(col, dtype=np.float32).reshape(N, C, k[0], k[1], OH, OW)
    for i in range(k[0]):
        for j in range(k[1]):
            hs, ws = i * d[0], j * d[1]
            padded[:, :, hs:hs + s[0] * (OH - 1) + 1:s[0],
                   ws:ws + s[1] * (OW - 1) + 1:s[1]] += c6[:, :, i, j]
    return padded[:, :, p[0]:p[0] + H, p[1]:p[1] + W]


@pytest.mark.parametrize("shape", [(2, 37, 100), (3, 1, 64), (5, 200, 49), (1, 3, 7), (4, 2048, 9)])
def test_zero_point_pos(shape):
    """atx_zero_point_pos against fp64: pos[n,l] = sum_o -(sx*sw[o])*zw[o]*go[n,o,l]
    (rel 1e-5 of the sum of |terms| + abs 1e-4), and bitwise equal run to run."""
    N, Oc, Lc = shape
    r = gen(zlib.crc32(repr(("zpp", shape)).encode()))
    go = r.standard_normal(shape).astype(np.float32)
    sx = np.float32(0.037)
    sw = (r.random(Oc) * 0.1 + 0.01).astype(np.float32)
    zw = r.integers(0, 16, Oc).astype(np.float32)
    coef = -((sx * sw).astype(np.float32) * zw).astype(np.float32)
    want = np.einsum("o,nol->nl", coef.astype(np.float64), go.astype(np.float64))
    bound = np.einsum("o,nol->nl", np.abs(coef).astype(np.float64), np.abs(go).astype(np.float64))
    a = ops.zero_point_pos(t(go), t(np.array(sx)), t(sw), t(zw))
    b = ops.zero_point_pos(t(go), t(np.array(sx)), t(sw), t(zw))
    assert torch.equal(a, b)
    close(a.cpu().numpy(), want, bound)


@pytest.mark.parametrize("shape", [(2, 37, 100), (3, 1, 64), (5, 200, 49), (1, 3, 7), (4, 2048, 9),
                                   (3, 130, 30), (64, 20, 3136), (2, 5000, 20), (2, 4, 0)])
@pytest.mark.parametrize("want_pos", [True, False])
def test_zero_point_terms(shape, want_pos):
    """atx_zero_point_terms: pos equal bit for bit to atx_zero_point_pos and
    gsum[o] = sum_{n,l} go[n,o,l] against fp64 (rel 1e-5 of the sum of
    |terms| + abs 1e-4), both identical run to run.  Shapes: 64- and
    16-position blocks (L >= 64 / < 64), channel counts that are not a
    multiple of a group's eight loads, more position blocks than workgroups
    (each walks several), more than 4096 channels, and L = 0 (zero sums)."""
    N, Oc, Lc = shape
    r = gen(zlib.crc32(repr(("zpt", shape)).encode()))
    go = r.standard_normal(shape).astype(np.float32)
    sx = np.float32(0.037)
    sw = (r.random(Oc) * 0.1 + 0.01).astype(np.float32)
    zw = r.integers(0, 16, Oc).astype(np.float32)
    args = (t(go), t(np.array(sx)), t(sw), t(zw))
    pos, gsum = ops.zero_point_terms(*args, want_pos=want_pos)
    pos2, gsum2 = ops.zero_point_terms(*args, want_pos=want_pos)
    assert torch.equal(gsum, gsum2)
    want = go.astype(np.float64).sum(axis=(0, 2))
    close(gsum.cpu().numpy(), want, np.abs(go).astype(np.float64).sum(axis=(0, 2)))
    if want_pos:
        assert torch.equal(pos, pos2)
        assert torch.equal(pos, ops.zero_point_pos(*args))
    else:
        assert pos is None


@pytest.mark.parametrize("case", TAP_GEOMS)
@pytest.mark.parametrize("dtype", ["uint8", "float32"])
def test_tap_sum_exact(case, dtype):
    """Column sums of the unfolded image with out-of-image taps counting as
    the zero point (nn/Conv2d_uint8.py:308-315): exact integers."""
    shape, k, s_, p, d = case
    r = gen(zlib.crc32(repr((case, dtype)).encode()))
    img = r.integers(0, 256, shape, dtype=np.uint8)
    z = np.float32(37.0)
    g = ops.conv_geom(shape, k, s_, p, d)
    src = t(img) if dtype == "uint8" else t(img.astype(np.float32))
    got = ops.tap_sum(src, g, pad_dev=t(np.array([z], np.float32)))
    want = O.im2col_index(img, k, s_, p, d, int(z)).astype(np.int64).sum(axis=1)
    assert np.array_equal(got.cpu().numpy(), want.astype(np.float32))


@pytest.mark.parametrize("shape", [(2, 130, 8, 12), (1, 64, 4, 4)])
def test_tap_sum_saturated(shape):
    """Byte images of 255 everywhere (H * W % 4 == 0: the 4-pixel kernel, whose
    16-bit fields then hold their largest sums, 64 * 255): exact."""
    img = np.full(shape, 255, dtype=np.uint8)
    z = np.float32(3.0)
    g = ops.conv_geom(shape, (3, 3), (1, 1), (1, 1), (1, 1))
    got = ops.tap_sum(t(img), g, pad_dev=t(np.array([z], np.float32)))
    want = O.im2col_index(img, (3, 3), (1, 1), (1, 1), (1, 1), int(z)).astype(np.int64).sum(axis=1)
    assert np.array_equal(got.cpu().numpy(), want.astype(np.float32))


CUSTOM_SHAPES = [(1, 1, 1, 1), (2, 5, 7, 3), (1, 4, 4096, 16), (3, 37, 1000, 70),
                 (2, 576, 3136, 64), (1, 9, 2049, 17), (4, 64, 49, 300), (1, 130, 6, 2048),
                 (2, 3, 5000, 33),
                 # L % 4 == 0 (resident tables): an odd number of tap quads (the last
                 # chunk holds one), one channel tile over many row steps (one slice
                 # per step), a partial last step with O % 16 != 0, row chunks of two
                 # steps, and one chunk of five steps whose rows cross images
                 (2, 9, 1024, 20), (2, 130, 12, 48), (5, 8, 4096, 16), (3, 18, 2500, 24),
                 (4, 144, 2600, 64), (2, 576, 4400, 48)]


@pytest.mark.parametrize("shape", CUSTOM_SHAPES)
def test_custom_grads_tiled_shapes(shape):
    """Pair-table gradients from the row-offset operand across row tiles (R
    above, below and one past 2048), channel tiles (O % 16 != 0, many
    tiles), tap quads (K % 4 != 0) and L % 4 != 0, with the fused
    per-channel STE on grad_w; against the fp64 C oracle within the sum of
    |terms| bound."""
    N, K, Lc, Oc = shape
    r = gen(zlib.crc32(repr(("custom", shape)).encode()))
    xi = r.integers(0, 256, (N, K, Lc), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    dxl = r.standard_normal(65536).astype(np.float32)
    dwl = r.standard_normal(65536).astype(np.float32)
    go = r.standard_normal((N, Oc, Lc)).astype(np.float32)
    mask = r.random((Oc, K)) < 0.8
    scale = (r.random(Oc) + 0.5).astype(np.float32)
    gx, gw = ops.custom_grads(ops.pack_rows_u8(t(xi)), t(wi), t(go), t(dxl), t(dwl), N, K, Lc,
                              mask_w=t(mask), scale_w=t(scale))
    ex, ew = O.gemm_grads(go, xi, wi, "custom", (dxl, dwl))
    ax, aw = O.gemm_grads(go, xi, wi, "custom", (dxl, dwl), absolute=True)
    close(gx.cpu().numpy(), ex, ax)
    ew = np.where(mask, ew, 0.0) / scale[:, None]
    aw = np.where(mask, aw, 0.0) / scale[:, None]
    close(gw.cpu().numpy(), ew, aw)


@pytest.mark.parametrize("case", TAP_GEOMS)
def test_col2im_pos_ste(case):
    """col2im with the per-position term (tap_sum's backward) and the fused
    STE: fold(col) + fold(pos broadcast over the taps of each position), then
    (mask ? v : 0) / scale, against the fp64 oracle fold."""
    shape, k, s_, p, d = case
    N, C, H, W = shape
    r = gen(zlib.crc32(repr(("col2im_pos", case)).encode()))
    g = ops.conv_geom(shape, k, s_, p, d)
    Lc = g.OH * g.OW
    col = r.standard_normal((N, C * k[0] * k[1], Lc)).astype(np.float32)
    pos = r.standard_normal((N, Lc)).astype(np.float32)
    mask = r.random(shape) < 0.7
    scale = np.float32(0.37)
    got = ops.col2im(t(col), g, pos=t(pos), mask=t(mask), scale=t(np.array([scale])))
    fcol = O.fold(col, shape, k, s_, p, d)
    fpos = O.fold(np.broadcast_to(pos[:, None, :], col.shape), shape, k, s_, p, d)
    want = np.where(mask, fcol + fpos, 0.0) / scale
    absref = np.where(mask, O.fold(np.abs(col), shape, k, s_, p, d) +
                      O.fold(np.abs(np.broadcast_to(pos[:, None, :], col.shape)), shape, k, s_,
                             p, d), 0.0) / scale
    close(got.cpu().numpy(), want, absref)
    plain = ops.col2im(t(col), g)
    close(plain.cpu().numpy(), fcol, O.fold(np.abs(col), shape, k, s_, p, d))
    # bit for bit: the fp32 sums in ascending tap order, the position sum
    # added once, then the STE's select and division in fp32
    f32col = fold_f32(col, shape, k, s_, p, d)
    f32pos = fold_f32(np.broadcast_to(pos[:, None, :], col.shape), shape, k, s_, p, d)
    exact = np.where(mask, f32col + f32pos, np.float32(0)) / np.maximum(scale, np.float32(1e-12))
    assert exact.dtype == np.float32
    assert np.array_equal(got.cpu().numpy(), exact)
    assert np.array_equal(plain.cpu().numpy(), f32col)


@pytest.mark.parametrize("shape", CUSTOM_SHAPES[:4] + [(2, 72, 3136, 64), (3, 40, 49, 70)])
def test_custom_grad_dw_uint8_zero_point(shape):
    """atx_custom_grad_dw_uint8: the uint8 layer's weight zero-point term
    (go_sum[o] * (scale_x * scale_w[o])) * zero_x subtracted in grad_w's slice
    sum, then the weight STE, equals the custom grad_w followed by the same
    torch expressions the layer used before (gw -= (gsum * (sx * sw)) * zx;
    (mask ? gw : 0) / max(sw, 1e-12)) bit for bit (resident-table and
    per-row-tile forms)."""
    N, K, Lc, Oc = shape
    r = gen(zlib.crc32(repr(("custom_u8zp", shape)).encode()))
    xi = r.integers(0, 256, (N, K, Lc), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    dwl = r.standard_normal(65536).astype(np.float32)
    go = t(r.standard_normal((N, Oc, Lc)).astype(np.float32))
    mask = t(r.random((Oc, K)) < 0.8)
    sw = t((r.random(Oc) * 0.05 + 0.01).astype(np.float32))
    sx = t(np.array([0.043], np.float32))
    zx = t(np.array([37.0], np.float32))
    gsum = go.sum(dim=(0, 2))
    c = (sx * sw).contiguous()
    op = ops.pack_rows_u8(t(xi))
    _, a = ops.custom_grads(op, t(wi), go, None, t(dwl), N, K, Lc, dy_scale=c, mask_w=mask,
                            scale_w=sw, w_zero_point=(gsum, sx, zx))
    _, b = ops.custom_grads(op, t(wi), go, None, t(dwl), N, K, Lc, dy_scale=c)
    b -= (gsum * c).mul_(zx).view(-1, 1)
    b = ops.fakequant_per_tensor_backward(b, mask, sw, channels=Oc, inner=K)
    assert torch.equal(a, b)


NARROW_SHAPES = CUSTOM_SHAPES +[(2, 64, 3136, 256), (3, 4608, 49, 40), (2, 20, 196, 2048)]


@pytest.mark.parametrize("shape", NARROW_SHAPES)
@pytest.mark.parametrize("wbase", [0, 120, 240])
def test_custom_grad_dx_narrow(shape, wbase):
    """grad_x of weights with 16 distinct indices on the matrix cores
    (atx_custom_grad_dx_narrow): row tiles of 256 (R not a multiple), tap
    tiles of 16 (K % 16 != 0), 32-channel steps (O % 32 != 0) and L % 16 != 0
    (row blocks across images), against the fp64 C oracle within the sum of
    |terms| bound; wbase 120 is the int8 weight_bits = 4 range v + 128."""
    N, K, Lc, Oc = shape
    r = gen(zlib.crc32(repr(("narrow", shape, wbase)).encode()))
    xi = r.integers(0, 256, (N, K, Lc), dtype=np.uint8)
    wi = r.integers(wbase, wbase + 16, (Oc, K), dtype=np.uint8)
    dxl = r.standard_normal(65536).astype(np.float32)
    go = r.standard_normal((N, Oc, Lc)).astype(np.float32)
    go[:, ::7] *= 1e-3                    # spread of magnitudes (three-part split)
    gx, _ = ops.custom_grads(ops.pack_rows_u8(t(xi)), t(wi), t(go), t(dxl), None, N, K, Lc,
                             wbase=wbase)
    ex, _ = O.gemm_grads(go, xi, wi, "custom", (dxl, dxl))
    ax, _ = O.gemm_grads(go, xi, wi, "custom", (dxl, dxl), absolute=True)
    close(gx.cpu().numpy(), ex, ax)


@pytest.mark.parametrize("shape", [(2, 37, 1000, 70), (1, 9, 2049, 17), (2, 64, 196, 300)])
def test_custom_grads_dy_scale(shape):
    """dy_scale[o] inside the kernels gives the gradients of the scaled copy
    dy * dy_scale[o] bit for bit (the same rounded products): grad_w of the
    pair-table kernel and grad_x of the matrix-core kernel."""
    N, K, Lc, Oc = shape
    r = gen(zlib.crc32(repr(("dys", shape)).encode()))
    xi = r.integers(0, 256, (N, K, Lc), dtype=np.uint8)
    wi = r.integers(0, 16, (Oc, K), dtype=np.uint8)
    tb = t(r.standard_normal(65536).astype(np.float32))
    go = t(r.standard_normal((N, Oc, Lc)).astype(np.float32))
    c = t((r.random(Oc) * 3e-3 + 1e-4).astype(np.float32))
    op = ops.pack_rows_u8(t(xi))
    a = ops.custom_grads(op, t(wi), go, tb, tb, N, K, Lc, wbase=0, dy_scale=c)
    b = ops.custom_grads(op, t(wi), go * c.view(1, -1, 1), tb, tb, N, K, Lc, wbase=0)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_custom_grad_dx_narrow_matches_general():
    """The matrix-core grad_x and the pair-table kernel agree within the fp32
    sum bound on a c5 layer shape (ResNet-50 3x3, 64 channels)."""
    N, K, Lc, Oc = 2, 576, 3136, 64
    r = gen(91)
    xi = r.integers(0, 256, (N, K, Lc), dtype=np.uint8)
    wi = r.integers(0, 16, (Oc, K), dtype=np.uint8)
    dxl = t(r.standard_normal(65536).astype(np.float32))
    go = t(r.standard_normal((N, Oc, Lc)).astype(np.float32))
    op = ops.pack_rows_u8(t(xi))
    a, _ = ops.custom_grads(op, t(wi), go, dxl, None, N, K, Lc, wbase=0)
    b, _ = ops.custom_grads(op, t(wi), go, dxl, None, N, K, Lc)
    ax, _ = O.gemm_grads(go.cpu().numpy(), xi, wi, "custom",
                         (dxl.cpu().numpy().reshape(256, 256),) * 2, absolute=True)
    close(a.cpu().numpy(), b.cpu().numpy(), 2 * ax)


@pytest.mark.parametrize("case", [(2, 40, (14, 14), 70, True, True), (1, 33, (25, 40), 16, False, True),
                                  (3, 16, (8, 8), 20, True, False), (2, 24, (10, 10), 32, False, False),
                                  (2, 8, (6, 6), 0, True, True)])
def test_custom_grad_dx_narrow_img_is_the_fold(case):
    """For a 1x1 stride-1 unpadded conv the matrix-core grad_x with the
    zero-point position term and the fake-quant STE in its epilogue
    (atx_custom_grad_dx_narrow_img) equals grad_x followed by the fold with
    them (atx_col2im_pos) bit for bit; O = 0 gives the fold of zeros."""
    N, C, (H, W), Oc, with_pos, with_mask = case
    Lc = H * W
    r = gen(zlib.crc32(repr(("img", case)).encode()))
    xi = r.integers(0, 256, (N, C, Lc), dtype=np.uint8)
    wi = r.integers(0, 16, (Oc, C), dtype=np.uint8)
    dxl = t(r.standard_normal(65536).astype(np.float32))
    go = t(r.standard_normal((N, Oc, Lc)).astype(np.float32))
    c = t((r.random(Oc) * 3e-3 + 1e-4).astype(np.float32))
    pos = t(r.standard_normal((N, Lc)).astype(np.float32)) if with_pos else None
    mask = t(r.random((N, C, H, W)) < 0.8) if with_mask else None
    sc = t(np.array([0.037], np.float32))
    g = ops.conv_geom((N, C, H, W), 1, 1, 0, 1)
    op = ops.pack_rows_u8(t(xi))
    a, _ = ops.custom_grads(op, t(wi), go, dxl, None, N, C, Lc, wbase=0, dy_scale=c,
                            img_ste=(pos, mask, sc))
    col, _ = ops.custom_grads(op, t(wi), go, dxl, None, N, C, Lc, wbase=0, dy_scale=c)
    b = ops.col2im(col, g, pos=pos, mask=mask, scale=sc)
    assert torch.equal(a.view_as(b), b)


def test_custom_grads_deterministic():
    """The grad_w partial slices are summed in a fixed order: two runs agree bitwise."""
    N, K, Lc, Oc = 4, 288, 3136, 64
    r = gen(77)
    xi = r.integers(0, 256, (N, K, Lc), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    tb = t(r.standard_normal(65536).astype(np.float32))
    go = t(r.standard_normal((N, Oc, Lc)).astype(np.float32))
    op = ops.pack_rows_u8(t(xi))
    a = ops.custom_grads(op, t(wi), go, tb, tb, N, K, Lc)
    b = ops.custom_grads(op, t(wi), go, tb, tb, N, K, Lc)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("geom", GEOMS)
def test_conv_backward_kernels(geom):
    k, s, p, d = geom
    r = gen(51)
    img = r.integers(-127, 128, (2, 6, 12, 13)).astype(np.int8)
    Oc = 20
    K = 6 * k[0] * k[1]
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    g = ops.conv_geom(img.shape, k, s, p, d)
    go = r.standard_normal((2, Oc, g.OH * g.OW)).astype(np.float32)
    tx = r.standard_normal(256).astype(np.float32)
    tw = r.standard_normal(256).astype(np.float32)
    gi = ops.conv_backward_data(t(go), t(wi), t(tx), g)
    gwk = ops.conv_backward_weight(t(go), t(img), t(tw), g, Oc, 128)
    xi = O.im2col_index(O.image_index(img), k, s, p, d, 128)
    ex, ew = O.gemm_grads(go, xi, wi, "lre", (tx, tw))
    close(gi.cpu().numpy(), O.fold(ex, img.shape, k, s, p, d))
    close(gwk.cpu().numpy(), ew)


@pytest.mark.parametrize("exact_tables", [False, True])
@pytest.mark.parametrize("where", ["go", "tables"])
def test_conv_backward_non_finite_operands(exact_tables, where):
    """+-inf and NaN in the output gradient, or in the tables, against the
    fp64 oracle.  Non-finite go: the bf16-split products are non-finite
    exactly where the oracle is (fp32's set of non-finite gradients).
    Non-finite table entries: every gradient the oracle makes non-finite is
    non-finite here too, but a tile's masked contraction terms (go zeroed, the
    table entry kept) can add 0 * inf = NaN to other gradients of that tile,
    so only "some gradient is non-finite" is fp32's.  Either way a finite
    result matches the oracle within the tolerance, and a six-product result
    may be NaN where fp32 gives +-inf (a part product inf * 0)."""
    k, s, p, d = (3, 3), (1, 1), (1, 1), (1, 1)
    r = gen(57)
    img = r.integers(-127, 128, (2, 6, 12, 13)).astype(np.int8)
    Oc, K = 20, 6 * 9
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    g = ops.conv_geom(img.shape, k, s, p, d)
    go = r.standard_normal((2, Oc, g.OH * g.OW)).astype(np.float32)
    if exact_tables:
        tx = r.integers(-100, 100, 256).astype(np.float32)
        tw = r.integers(-100, 100, 256).astype(np.float32)
    else:
        tx = r.standard_normal(256).astype(np.float32)
        tw = r.standard_normal(256).astype(np.float32)
    if where == "go":
        go[0, 3, 17], go[1, 11, 40], go[1, 5, 99] = np.inf, -np.inf, np.nan
    else:
        tx[int(wi[7, 30])] = np.inf
        tw[200] = -np.inf
    gi = ops.conv_backward_data(t(go), t(wi), t(tx), g).cpu().numpy()
    gwk = ops.conv_backward_weight(t(go), t(img), t(tw), g, Oc, 128).cpu().numpy()
    xi = O.im2col_index(O.image_index(img), k, s, p, d, 128)
    with np.errstate(invalid="ignore", over="ignore"):
        tabs = (tx.astype(np.float64), tw.astype(np.float64))
        ex, ew = O.gemm_grads(go.astype(np.float64), xi, wi, "lre", tabs)
        ax, aw = O.gemm_grads(go.astype(np.float64), xi, wi, "lre", tabs, absolute=True)
        exi = O.fold(ex, img.shape, k, s, p, d)
        axi = O.fold(ax, img.shape, k, s, p, d)
    for got, want, bound in ((gi, exi, axi), (gwk, ew, aw)):
        fin, gfin = np.isfinite(want), np.isfinite(got)
        assert (~fin).any() and fin.any()
        if where == "go":
            assert np.array_equal(gfin, fin)
        else:
            assert not (gfin & ~fin).any() and (~gfin).any()
        both = fin & gfin
        close(got[both], want[both], bound[both])


# (image shape, (kernel, stride, padding, dilation), O, image dtype): multi-tile
# backward GEMMs over 64- and 128-wide tiles, partial tiles, L % 4 != 0
# (scalar operand loads), K % 4 != 0, split contractions and every image type.
BWD_TILED = [
    ((2, 64, 14, 14), ((3, 3), (1, 1), (1, 1), (1, 1)), 128, "int8"),
    ((3, 32, 7, 7), ((1, 1), (1, 1), (0, 0), (1, 1)), 64, "uint8"),
    ((2, 16, 9, 11), ((3, 3), (2, 2), (1, 1), (1, 1)), 200, "float32"),
    ((1, 3, 20, 20), ((5, 5), (1, 1), (2, 2), (1, 1)), 70, "int8"),
    ((4, 128, 8, 8), ((1, 1), (1, 1), (0, 0), (1, 1)), 256, "uint8"),
    ((8, 64, 28, 28), ((1, 1), (2, 2), (0, 0), (1, 1)), 96, "int8"),
]


@pytest.mark.parametrize("case", BWD_TILED)
def test_conv_backward_kernels_tiled(case):
    shape, (k, s, p, d), Oc, dtype = case
    r = gen(zlib.crc32(repr(case).encode()))
    if dtype == "int8":
        img = r.integers(-128, 128, shape).astype(np.int8)
    elif dtype == "uint8":
        img = r.integers(0, 256, shape).astype(np.uint8)
    else:
        img = r.integers(-130, 130, shape).astype(np.float32)
    K = shape[1] * k[0] * k[1]
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    g = ops.conv_geom(img.shape, k, s, p, d)
    go = r.standard_normal((shape[0], Oc, g.OH * g.OW)).astype(np.float32)
    tx = r.standard_normal(256).astype(np.float32)
    tw = r.standard_normal(256).astype(np.float32)
    pad = 128 if dtype != "uint8" else 7
    gi = ops.conv_backward_data(t(go), t(wi), t(tx), g)
    gwk = ops.conv_backward_weight(t(go), t(img), t(tw), g, Oc, pad)
    xi = O.im2col_index(O.image_index(img, 128), k, s, p, d, pad)
    ex, ew = O.gemm_grads(go, xi, wi, "lre", (tx, tw))
    ax, aw = O.gemm_grads(np.abs(go), xi, wi, "lre", (np.abs(tx), np.abs(tw)))
    close(gi.cpu().numpy(), O.fold(ex, img.shape, k, s, p, d), O.fold(ax, img.shape, k, s, p, d))
    close(gwk.cpu().numpy(), ew, aw)


@pytest.mark.parametrize("geom,shape,Oc", [
    (GEOMS[0], (3, 40, 11, 12), 72), (((1, 1), (1, 1), (0, 0), (1, 1)), (3, 40, 11, 12), 72),
    (GEOMS[2], (3, 40, 11, 12), 72),
    # few output tiles and a long contraction: split into partial slices
    (((1, 1), (1, 1), (0, 0), (1, 1)), (2, 96, 7, 7), 512), (GEOMS[0], (2, 32, 7, 7), 520),
    # the same with L % 4 == 0: partial slices written as 16-byte column quads
    (((1, 1), (1, 1), (0, 0), (1, 1)), (2, 96, 8, 8), 512), (GEOMS[0], (2, 32, 8, 8), 520),
    # stride 1 with O % 32 == 0 but few image tiles: col path
    (GEOMS[0], (3, 40, 11, 12), 64), (((5, 5), (1, 1), (0, 0), (1, 1)), (1, 8, 12, 9), 256),
    # stride 1, O % 32 == 0 and >= 512 image tiles: implicit backward-data GEMM
    (GEOMS[0], (2, 8, 128, 256), 32), (((3, 3), (1, 1), (2, 2), (2, 2)), (1, 8, 256, 257), 96),
    (((3, 1), (1, 1), (1, 0), (1, 1)), (1, 130, 256, 129), 32),
    (((5, 5), (1, 1), (0, 0), (1, 1)), (4, 4, 132, 131), 64)])
@pytest.mark.parametrize("exact", [False, True])
def test_conv_backward_fused_scale_and_masks(geom, shape, Oc, exact):
    """The fused layer backward: go * fp32(sx * sw[o]) in the operand loads,
    the x fake-quant STE (mask ? g : 0) / max(sx, 1e-12) on the image gradient
    (fold, or the GEMM epilogue of the 1x1 stride-1 conv), the per-channel W
    STE in the split-K sum.  exact: integer-valued tables (the STE's), whose
    bf16 split has only its high part (three part products per product)."""
    k, s, p, d = geom
    r = gen(zlib.crc32(repr((geom, shape, Oc)).encode()) + 7)
    img = r.integers(-127, 128, shape).astype(np.int8)
    K = shape[1] * k[0] * k[1]
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    g = ops.conv_geom(img.shape, k, s, p, d)
    go = r.standard_normal((shape[0], Oc, g.OH * g.OW)).astype(np.float32)
    if exact:
        tx = (np.arange(256) - 128).astype(np.float32)
        tw = r.permutation(tx)
    else:
        tx = r.standard_normal(256).astype(np.float32)
        tw = r.standard_normal(256).astype(np.float32)
    sx = np.array([0.0213], np.float32)
    sw = r.uniform(1e-3, 4e-2, Oc).astype(np.float32)
    mask_x = r.random(img.shape) < 0.9
    mask_w = r.random((Oc, K)) < 0.9
    gi = ops.conv_backward_data(t(go), t(wi), t(tx), g, mask=t(mask_x), scale=t(sx),
                                go_sx=t(sx), go_sw=t(sw))
    gwk = ops.conv_backward_weight(t(go), t(img), t(tw), g, Oc, 128, mask_w=t(mask_w),
                                   scale_w=t(sw), go_sx=t(sx), go_sw=t(sw))
    gos = go * (sx[0] * sw)[None, :, None]            # fp32 product, then fp32 scale
    xi = O.im2col_index(O.image_index(img), k, s, p, d, 128)
    ex, ew = O.gemm_grads(gos, xi, wi, "lre", (tx, tw))
    ax, aw = O.gemm_grads(np.abs(gos), xi, wi, "lre", (np.abs(tx), np.abs(tw)))
    fx = O.fold(ex, img.shape, k, s, p, d)
    fa = O.fold(ax, img.shape, k, s, p, d)
    ex_img = np.where(mask_x, fx, 0.0) / max(float(sx[0]), 1e-12)
    close(gi.cpu().numpy(), ex_img, fa / float(sx[0]))
    ew_m = np.where(mask_w, ew, 0.0) / np.maximum(sw, 1e-12)[:, None]
    close(gwk.cpu().numpy(), ew_m, aw / sw[:, None])


# ------------------------------------------------------------ depthwise conv
DW_GEOMS = [((3, 3), (1, 1), (1, 1), (1, 1)), ((3, 3), (2, 2), (1, 1), (1, 1)),
            ((5, 5), (1, 1), (2, 2), (1, 1)), ((7, 7), (2, 2), (3, 3), (1, 1)),
            ((3, 3), (1, 1), (2, 2), (2, 2)), ((3, 1), (1, 2), (1, 0), (1, 1))]


@pytest.mark.parametrize("geom", DW_GEOMS)
@pytest.mark.parametrize("dtype", ["int8", "uint8", "float32"])
def test_dwconv_fake_int8_claude(geom, dtype):
    """y = per-channel LUT conv (exact int64 oracle), out-of-image taps row 128,
    and wq = clamp(rint(w) + 128)."""
    k, s, p, d = geom
    r = gen(zlib.crc32(repr((geom, dtype)).encode()))
    C = 24
    if dtype == "int8":
        img = r.integers(-128, 128, (3, C, 15, 14)).astype(np.int8)
    elif dtype == "uint8":
        img = r.integers(0, 256, (3, C, 15, 14)).astype(np.uint8)
    else:
        img = r.integers(-130, 130, (3, C, 15, 14)).astype(np.float32)
    w = r.integers(-128, 128, (C, k[0] * k[1])).astype(np.float32)
    lut = luts(5)["perturbed"]
    y, wq = ops.dwconv_fake_int8_claude(t(img), t(w), t(lut, torch.float32), k, s, p, d)
    xi = O.image_index(img, 128)
    wi = (w + 128).astype(np.uint8)
    assert np.array_equal(wq.cpu().numpy(), wi)
    want = np.concatenate([O.lut_gemm_i64(O.im2col_index(xi[:, c:c + 1], k, s, p, d, 128),
                                          wi[c:c + 1], lut) for c in range(C)], axis=1)
    OH, OW = O.out_size(15, 14, k, s, p, d)
    assert y.shape == (3, C, OH, OW)
    assert np.array_equal(y.cpu().numpy().reshape(3, C, -1), want.astype(np.float32))


def test_pack_w_index_image_alone():
    """want_wt=False writes the same weight index image as the full pack
    (clamp(rint(w) + 128, 0, 255), halves to even, out-of-range values
    clamped) and no transposed operand."""
    r = gen(31)
    w = np.concatenate([r.integers(-140, 141, 200).astype(np.float32),
                        np.array([-0.5, 0.5, 1.5, 2.5, -127.5, 127.5], np.float32)])
    w = np.resize(w, (23, 9))
    wq, wt, Opad = ops._pack_w(t(w), 128, want_wt=False)
    assert wt is None and Opad == 32
    wq_full, wt_full, _ = ops._pack_w(t(w), 128)
    assert torch.equal(wq, wq_full)
    assert np.array_equal(wq.cpu().numpy(), O.quant_index(w, 128))
    assert np.array_equal(wt_full.cpu().numpy()[:, :23], O.quant_index(w, 128).T)


def misaligned(a):
    """a copied to the device at a byte address that is 1 mod 4 (a
    contiguous view one byte into a larger buffer)."""
    flat = np.ascontiguousarray(a).reshape(-1)
    buf = torch.empty(flat.size * flat.itemsize + 8, dtype=torch.uint8, device=DEV)
    v = buf[1:1 + flat.size * flat.itemsize].view(t(flat[:0]).dtype).view(a.shape)
    v.copy_(t(a))
    assert v.data_ptr() % 4 == 1
    return v


@pytest.mark.parametrize("aligned", [True, False])
@pytest.mark.parametrize("stride", [1, 2])
@pytest.mark.parametrize("hw", [(16, 16), (9, 31), (1, 4), (5, 8)])
@pytest.mark.parametrize("dtype", ["int8", "uint8"])
def test_dwconv_strips(stride, hw, dtype, aligned):
    """The 4-output strip kernels (3-wide kernels, stride 1 or 2 along W):
    OW a multiple of 4 (16-byte stores), ragged strips, a single row; a
    4-byte aligned image takes the 3x3 kernel reading rows as aligned dwords
    (W % 4 == 0 or not), a misaligned one the per-byte strip kernel; exact
    against the per-channel int64 oracle, the int32 output too."""
    H, W = hw
    k, s, p, d = (3, 3), (stride, stride), (1, 1), (1, 1)
    r = gen(zlib.crc32(repr(("strips", stride, hw, dtype)).encode()))
    C = 6
    if dtype == "int8":
        img = r.integers(-128, 128, (2, C, H, W)).astype(np.int8)
    else:
        img = r.integers(0, 256, (2, C, H, W)).astype(np.uint8)
    w = r.integers(-128, 128, (C, 9)).astype(np.float32)
    lut = luts(7)["asym"]
    img_d = t(img) if aligned else misaligned(img)
    y, wq = ops.dwconv_fake_int8_claude(img_d, t(w), t(lut, torch.float32), k, s, p, d)
    xi = O.image_index(img, 128)
    wi = (w + 128).astype(np.uint8)
    want = np.concatenate([O.lut_gemm_i64(O.im2col_index(xi[:, c:c + 1], k, s, p, d, 128),
                                          wi[c:c + 1], lut) for c in range(C)], axis=1)
    assert np.array_equal(y.cpu().numpy().reshape(2, C, -1), want.astype(np.float32))
    g = ops.conv_geom(img.shape, k, s, p, d)
    yi = torch.empty((2, C, g.OH, g.OW), dtype=torch.int32, device=DEV)
    img16, imgf, cls = ops.lut_image(t(lut, torch.float32))
    ep = LB.GemmEpilogue(LB.ATX_OUT_I32)
    LB.call("atx_dwconv_fwd", LB.ptr(img_d), 0 if dtype == "int8" else 1, g, 128, LB.ptr(wq),
            LB.ptr(img16), LB.ptr(imgf), cls, ep, LB.ptr(yi), LB.stream_of(yi))
    assert np.array_equal(yi.cpu().numpy().reshape(2, C, -1), want)


@pytest.mark.parametrize("case", [((2, 3, 1, 2), (1, 1), (1, 3)), ((2, 3, 1, 2), (1, 2), (2, 4)),
                                  ((3, 4, 15, 14), (1, 1), (1, 1)), ((2, 2, 5, 9), (2, 2), (1, 1)),
                                  ((4, 1, 2, 2), (1, 1), (1, 4))])
@pytest.mark.parametrize("dtype", ["int8", "uint8"])
def test_dwconv_strip_windows_before_the_image(case, dtype):
    """Rows whose dword window starts before the image's first byte (the
    first plane's top-left strips, and planes smaller than the padding,
    where later planes' windows start in an earlier plane) and windows past
    its last byte: exact against the int64 oracle through the 3x3 strip
    kernel."""
    shape, s, p = case
    k, d = (3, 3), (1, 1)
    r = gen(zlib.crc32(repr(("windows", case, dtype)).encode()))
    lo, hi = (-128, 128) if dtype == "int8" else (0, 256)
    img = r.integers(lo, hi, shape).astype(np.int8 if dtype == "int8" else np.uint8)
    C = shape[1]
    w = r.integers(-128, 128, (C, 9)).astype(np.float32)
    lut = luts(9)["asym"]
    y, _ = ops.dwconv_fake_int8_claude(t(img), t(w), t(lut, torch.float32), k, s, p, d)
    xi = O.image_index(img, 128)
    wi = (w + 128).astype(np.uint8)
    want = np.concatenate([O.lut_gemm_i64(O.im2col_index(xi[:, c:c + 1], k, s, p, d, 128),
                                          wi[c:c + 1], lut) for c in range(C)], axis=1)
    assert np.array_equal(y.cpu().numpy().reshape(shape[0], C, -1), want.astype(np.float32))


@pytest.mark.parametrize("geom", [((1, 1), (1, 1), (1, 1)), ((2, 2), (1, 1), (1, 1)),
                                  ((1, 2), (2, 0), (2, 1)), ((3, 1), (0, 3), (1, 1))])
@pytest.mark.parametrize("dtype", ["int8", "uint8"])
def test_dwconv_strip_groups(geom, dtype):
    """MobileNet-sized depthwise convs (64 x 64 x 112 x 112, 3x3), where each
    thread of the 3x3 strip kernel walks many groups of strips (positions
    advanced incrementally, the next group's rows read before the current
    one is summed): the aligned image (3x3 kernel) and the same image at a
    misaligned address (per-byte strip kernel) give identical outputs, and
    two channels match the int64 oracle; stride, padding and dilation along
    H differ from those along W."""
    s, p, d = geom
    k = (3, 3)
    r = gen(zlib.crc32(repr(("strip groups", geom, dtype)).encode()))
    N, C, H, W = 64, 64, 112, 112
    lo, hi = (-128, 128) if dtype == "int8" else (0, 256)
    img = r.integers(lo, hi, (N, C, H, W)).astype(np.int8 if dtype == "int8" else np.uint8)
    w = r.integers(-128, 128, (C, 9)).astype(np.float32)
    lut = t(luts(8)["asym"], torch.float32)
    y, wq = ops.dwconv_fake_int8_claude(t(img), t(w), lut, k, s, p, d)
    ym, _ = ops.dwconv_fake_int8_claude(misaligned(img), t(w), lut, k, s, p, d)
    assert torch.equal(y, ym)
    xi = O.image_index(img, 128)
    wi = (w + 128).astype(np.uint8)
    yc = y.cpu().numpy()
    for c in (0, C - 1):
        want = O.lut_gemm_i64(O.im2col_index(xi[:, c:c + 1], k, s, p, d, 128), wi[c:c + 1],
                              luts(8)["asym"])
        assert np.array_equal(yc[:, c].reshape(N, -1), want[:, 0].astype(np.float32))


@pytest.mark.parametrize("lut_name", ["u16_c5", "fp32"])
def test_dwconv_lut_classes(lut_name):
    r = gen(21)
    k, s, p, d = DW_GEOMS[0]
    img = r.integers(-128, 128, (2, 9, 10, 11)).astype(np.int8)
    w = r.integers(-128, 128, (9, 9)).astype(np.float32)
    xi = O.im2col_index(O.image_index(img, 128), k, s, p, d, 128)
    wi = (w + 128).astype(np.uint8)
    if lut_name == "fp32":
        lut = (r.standard_normal(65536) * 3).astype(np.float32)
        want = np.concatenate([O.lut_gemm_f32(xi[:, 9 * c:9 * c + 9], wi[c:c + 1], lut)
                               for c in range(9)], axis=1)
        y, _ = ops.dwconv_fake_int8_claude(t(img), t(w), t(lut), k, s, p, d)
        assert np.array_equal(y.cpu().numpy().reshape(2, 9, -1), want)
    else:
        lut = luts(5)[lut_name]
        want = np.concatenate([O.lut_gemm_i64(xi[:, 9 * c:9 * c + 9], wi[c:c + 1], lut)
                               for c in range(9)], axis=1)
        y, _ = ops.dwconv_fake_int8_claude(t(img), t(w), t(lut, torch.float32), k, s, p, d)
        assert np.array_equal(y.cpu().numpy().reshape(2, 9, -1), want.astype(np.float32))


@pytest.mark.parametrize("geom", DW_GEOMS)
def test_dwconv_backward_kernels(geom):
    """Per-channel table gradients (gemm_grads + fold per channel) with the
    go scale and both fake-quant STE masks fused."""
    k, s, p, d = geom
    r = gen(zlib.crc32(repr(geom).encode()) + 3)
    C = 20
    img = r.integers(-127, 128, (3, C, 13, 12)).astype(np.int8)
    wi = r.integers(0, 256, (C, k[0] * k[1]), dtype=np.uint8)
    g = ops.conv_geom(img.shape, k, s, p, d)
    go = r.standard_normal((3, C, g.OH, g.OW)).astype(np.float32)
    tx = r.standard_normal(256).astype(np.float32)
    tw = r.standard_normal(256).astype(np.float32)
    sx = np.array([0.031], np.float32)
    sw = r.uniform(1e-3, 4e-2, C).astype(np.float32)
    mask_x = r.random(img.shape) < 0.9
    mask_w = r.random(wi.shape) < 0.9
    gi = ops.dwconv_backward_data(t(go), t(wi), t(tx), g, mask=t(mask_x), scale=t(sx),
                                  go_sx=t(sx), go_sw=t(sw)).cpu().numpy()
    gwk = ops.dwconv_backward_weight(t(go), t(img), t(tw), g, 128, mask_w=t(mask_w),
                                     scale_w=t(sw), go_sx=t(sx), go_sw=t(sw)).cpu().numpy()
    xi = O.image_index(img)
    for c in range(C):
        gos = go[:, c:c + 1].reshape(3, 1, -1) * (sx[0] * sw[c])
        xc = O.im2col_index(xi[:, c:c + 1], k, s, p, d, 128)
        ex, ew = O.gemm_grads(gos, xc, wi[c:c + 1], "lre", (tx, tw))
        ax, aw = O.gemm_grads(np.abs(gos), xc, wi[c:c + 1], "lre", (np.abs(tx), np.abs(tw)))
        shp = (3, 1, 13, 12)
        fx, fa = O.fold(ex, shp, k, s, p, d), O.fold(ax, shp, k, s, p, d)
        close(gi[:, c:c + 1], np.where(mask_x[:, c:c + 1], fx, 0.0) / float(sx[0]),
              fa / float(sx[0]))
        close(gwk[c:c + 1], np.where(mask_w[c:c + 1], ew, 0.0) / float(sw[c]), aw / float(sw[c]))


@pytest.mark.parametrize("case", BWD_TILED)
def test_conv_backward_weight_rows_equals_image_path(case):
    """The weight gradient from the forward's row-offset operand is the
    image-path result bit for bit (same tiles, same summation order)."""
    shape, (k, s, p, d), Oc, dtype = case
    r = gen(zlib.crc32(repr(case).encode()) + 11)
    if dtype == "int8":
        img = r.integers(-128, 128, shape).astype(np.int8)
        offset, pad = 128, 128
    elif dtype == "uint8":
        img = r.integers(0, 256, shape).astype(np.uint8)
        offset, pad = 0, 7
    else:
        img = r.integers(-130, 130, shape).astype(np.float32)
        offset, pad = 128, 128
    K = shape[1] * k[0] * k[1]
    w = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    g = ops.conv_geom(img.shape, k, s, p, d)
    lut = t(luts(2)["perturbed"], torch.float32)
    _, _, operand = ops.conv_forward(t(img), t(w), lut, g, offset, pad, return_operand=True)
    go = t(r.standard_normal((shape[0], Oc, g.OH * g.OW)).astype(np.float32))
    tw = t(r.standard_normal(256).astype(np.float32))
    sx = t(np.array([0.02], np.float32))
    sw = t(r.uniform(1e-3, 4e-2, Oc).astype(np.float32))
    a = ops.conv_backward_weight(go, t(img), tw, g, Oc, pad, go_sx=sx, go_sw=sw)
    b = ops.conv_backward_weight_rows(go, operand, tw, g, Oc, go_sx=sx, go_sw=sw)
    assert torch.equal(a, b)
