"""GPU parity of the LUT GEMM's upper-half tables (atx_gemm_epilogue.x_upper:
every activation index >= 128, as for the int8 operand of an x >= 0) and of
the flag that promises it (atx_absmax_ema_upper).

Bar: the int32 sums bit-exact against the int64 oracle and equal to the
full-table path; the statistic and the EMA scale bit for bit equal to
atx_absmax_ema's.  The promise is always kept here: a broken one gives wrong
sums by contract, which is not tested.
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


def gen(seed):
    return np.random.default_rng(seed)


def t(a, dtype=None):
    return torch.as_tensor(np.ascontiguousarray(a), device=DEV, dtype=dtype)


def lut_of(name, seed=3):
    r = gen(seed)
    v = np.arange(256)
    a = v - 128
    if name == "asym":                                   # catches swapped operands
        return (37 * v[:, None] - 19 * v[None, :] + 11).reshape(-1)
    if name == "u16":                                    # unsigned class
        return ((v[:, None] * v[None, :]) & ~63).reshape(-1)
    return np.clip((a[:, None] * a[None, :]) +             # signed class, perturbed
                   np.rint(r.normal(0, 1, (256, 256)) * (0.02 * np.abs(a[:, None] * a[None, :]) + 1)),
                   -32768, 32767).reshape(-1)


def flag(value):
    return torch.full((), value, dtype=torch.int32, device=DEV)


def gemm_i32(xi, wi, lut, x_upper):
    """lut_gemm_i32 with the x_upper flag passed to the kernel."""
    xc, wc = t(xi), t(wi)
    N, K, Lc = xc.shape
    Oc = wc.size(0)
    Rpad = LB.round_up(max(N * Lc, 1), LB.ROW_TILE)
    xt = torch.empty((LB.operand_rows(K), Rpad), dtype=torch.int16, device=DEV)
    LB.call("atx_pack_x_u8", LB.ptr(xc), N, K, Lc, LB.ptr(xt), Rpad, None, LB.stream_of(xc))
    _, wt, Opad = ops._pack_w(wc, 0)
    y = torch.empty((N, Oc, Lc), dtype=torch.int32, device=DEV)
    ops._gemm(xt, Rpad, wt, Opad, N, K, Lc, Oc, t(lut, torch.float32), LB.ATX_OUT_I32, y,
              x_upper=x_upper)
    return y.cpu().numpy().astype(np.int64)


# (N, K, L, O): K not a multiple of 4 (padding taps read table row 0), rows
# not a multiple of the tile (padding rows), O not a multiple of 32, one and
# several row tiles, short and long contractions.
SHAPES = [(1, 1, 1, 1), (2, 5, 7, 3), (3, 33, 9, 17), (2, 576, 64, 64), (1, 300, 1100, 65),
          (4, 64, 49, 130), (1, 4608, 49, 64), (8, 576, 1024, 64)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("lut_name", ["asym", "perturbed", "u16"])
def test_upper_tables_bit_exact(shape, lut_name):
    N, K, L, Oc = shape
    r = gen(zlib.crc32(repr(("upper", shape, lut_name)).encode()))
    xi = r.integers(128, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = lut_of(lut_name)
    want = O.lut_gemm_i64(xi, wi, lut)
    assert np.array_equal(gemm_i32(xi, wi, lut, flag(1)), want)
    # a zero flag or none: the full tables, same sums
    assert np.array_equal(gemm_i32(xi, wi, lut, flag(0)), want)
    assert np.array_equal(gemm_i32(xi, wi, lut, None), want)


@pytest.mark.parametrize("sched,rows,splits", [("stream_k", None, None), ("split", None, None),
                                                ("split", 1792, 1), ("split", 768, 3)])
def test_upper_tables_schedules(sched, rows, splits, monkeypatch):
    """Stream-K tails, split-K partials and short row tiles (waves past the
    tile build tables only) with upper-half tables."""
    monkeypatch.setenv("ATX_LUT_SCHEDULE", sched)
    if rows:
        monkeypatch.setenv("ATX_LUT_ROWS", str(rows))
        monkeypatch.setenv("ATX_LUT_SPLITS", str(splits))
    N, K, L, Oc = (1, 1000, 4096, 40) if sched == "stream_k" else (3, 301, 1100, 70)
    r = gen(zlib.crc32(repr(("upper-sched", sched, rows, splits)).encode()))
    xi = r.integers(128, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = lut_of("perturbed")
    assert np.array_equal(gemm_i32(xi, wi, lut, flag(1)), O.lut_gemm_i64(xi, wi, lut))


def test_upper_tables_noalloc_entry():
    """atx_lut_gemm_noalloc reads the same flag (shares the kernels)."""
    N, K, L, Oc = 2, 130, 700, 48
    r = gen(31)
    xi = r.integers(128, 256, (N, K, L), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = lut_of("asym")
    xc = t(xi)
    Rpad = LB.round_up(N * L, LB.ROW_TILE)
    xt = torch.empty((LB.operand_rows(K), Rpad), dtype=torch.int16, device=DEV)
    LB.call("atx_pack_x_u8", LB.ptr(xc), N, K, L, LB.ptr(xt), Rpad, None, LB.stream_of(xc))
    _, wt, Opad = ops._pack_w(t(wi), 0)
    img16, imgf, cls = ops.lut_image(t(lut, torch.float32))
    y = torch.empty((N, Oc, L), dtype=torch.int32, device=DEV)
    f = flag(1)
    ep = LB.GemmEpilogue(LB.ATX_OUT_I32, None, None, None, LB.ptr(f))
    LB.call("atx_lut_gemm_noalloc", LB.ptr(xt), Rpad, LB.ptr(wt), Opad, N, K, L, Oc,
            LB.ptr(img16), LB.ptr(imgf), cls, ep, LB.ptr(y), LB.stream_of(y))
    assert np.array_equal(y.cpu().numpy().astype(np.int64), O.lut_gemm_i64(xi, wi, lut))


def _stats(x, upper_entry):
    xc = x.contiguous()
    ws = ops._reduce_ws(x.device)
    stat = torch.empty((), dtype=torch.float32, device=DEV)
    scale = torch.full((), 0.37, dtype=torch.float32, device=DEV)
    m32, om32 = np.float32(0.1), np.float32(0.9)
    if upper_entry:
        up = torch.full((), -5, dtype=torch.int32, device=DEV)
        LB.call("atx_absmax_ema_upper", LB.ptr(xc), xc.numel(), LB.ptr(ws), LB.ptr(stat),
                127.0, float(m32), float(om32), LB.ptr(scale), LB.ptr(up), LB.stream_of(xc))
        return stat.item(), scale.item(), int(up.item())
    LB.call("atx_absmax_ema", LB.ptr(xc), xc.numel(), LB.ptr(ws), LB.ptr(stat), 127.0,
            float(m32), float(om32), LB.ptr(scale), LB.stream_of(xc))
    return stat.item(), scale.item(), None


@pytest.mark.parametrize("case", ["relu", "relu_negzero", "zeros", "one_negative", "nan",
                                  "inf", "randn", "large"])
def test_absmax_ema_upper_flag_and_bitwise_stat(case):
    r = gen(zlib.crc32(case.encode()))
    n = 300_001 if case == "large" else 5003
    x = np.maximum(r.standard_normal(n).astype(np.float32), 0)
    if case == "relu_negzero":
        x[::7] = -0.0
    elif case == "zeros":
        x[:] = 0.0
    elif case == "one_negative":
        x[r.integers(0, n)] = -1e-3
    elif case == "nan":
        x[r.integers(0, n)] = np.nan
    elif case == "inf":
        x[r.integers(0, n)] = np.inf
    elif case == "randn":
        x = r.standard_normal(n).astype(np.float32)
    xg = t(x)
    s_up, sc_up, up = _stats(xg, True)
    s_ref, sc_ref, _ = _stats(xg, False)
    # the statistic and the EMA scale are atx_absmax_ema's, bit for bit
    assert np.array_equal(np.float32(s_up), np.float32(s_ref), equal_nan=True)
    assert np.array_equal(np.float32(sc_up), np.float32(sc_ref), equal_nan=True)
    expect_up = bool(np.all(x >= 0))          # NaN compares false
    assert up == int(expect_up), (case, up)


class GemmSpy:
    """Records the x_upper flag value each LUT GEMM call saw."""

    def __init__(self, monkeypatch):
        self.seen = []
        orig = ops._gemm

        def spy(*a, **kw):
            out = orig(*a, **kw)
            up = kw.get("x_upper")
            self.seen.append(None if up is None else int(up.item()))
            return out
        monkeypatch.setattr(ops, "_gemm", spy)


def full_tables(monkeypatch):
    """Withholds every derived flag: the LUT GEMM builds full tables."""
    monkeypatch.setattr(ops, "upper_flag", lambda device: None)


def _full_table_forward(layer, x, kernel):
    from approxtorch_amd.nn import bgemm_int8
    qmax_w = 2 ** (layer.weight_bits - 1) - 1
    tx = tw = bgemm_int8.decode_table(x.device)
    geom = ((kernel, kernel), layer.stride, layer.padding, layer.dilation, layer.groups)
    return bgemm_int8.conv2d_int8_fused(x, layer.weight, layer.bias, layer.scale_x,
                                        layer.scale_w, layer.lut, tx, tw, geom, layer.qmin,
                                        layer.qmax, qmax_w).detach()


@pytest.mark.parametrize("kernel,pad", [(3, 1), (1, 0)])
def test_conv2d_int8_training_forward_with_upper_tables(kernel, pad, monkeypatch):
    """A train-mode Conv2d_int8 forward on a non-negative input (the flag is
    set, upper-half tables) equals the same layer's forward through the
    full tables (the flag withheld) and the oracle."""
    import approxtorch_amd as at
    torch.manual_seed(11)
    lut = t(lut_of("perturbed"), torch.float32)
    layer = at.nn.Conv2d_int8(16, 40, kernel, lut, grad="ste", bias=True, padding=pad).to(DEV)
    layer.train()
    x = torch.relu(torch.randn(3, 16, 13, 11, device=DEV))
    spy = GemmSpy(monkeypatch)
    y = layer(x).detach()
    assert spy.seen == [1]
    # the same fake-quant and conv with the full tables, at the updated scales
    with monkeypatch.context() as m:
        full_tables(m)
        y_full = _full_table_forward(layer, x, kernel)
    assert spy.seen[1:] == [None]
    assert torch.equal(y, y_full)
    sx = np.float32(layer.scale_x.item())
    sw = layer.scale_w.cpu().numpy()
    want, ctx = O.conv_int8_forward(x.cpu().numpy(), layer.weight.detach().cpu().numpy(),
                                    layer.bias.detach().cpu().numpy(), lut.cpu().numpy(), sx,
                                    sw, (kernel, kernel), (1, 1), (pad, pad), (1, 1))
    got = y.double().cpu().numpy()
    # rel 1e-5 of the sum of |terms| (ctx["yabs"]) plus abs 1e-4
    assert np.max(np.abs(got - want) - 1e-5 * ctx["yabs"]) <= 1e-4


@pytest.mark.parametrize("kernel,pad", [(3, 1), (1, 0)])
@pytest.mark.parametrize("relu", [True, False])
def test_conv2d_int8_eval_forward_upper_tables(kernel, pad, relu, monkeypatch):
    """Eval mode (no statistic): the fake-quant derives the flag from the
    quantized x (set for a ReLU input, cleared otherwise); the forward equals
    the full-table forward bit for bit and the oracle within tolerance."""
    import approxtorch_amd as at
    torch.manual_seed(13)
    lut = t(lut_of("perturbed"), torch.float32)
    layer = at.nn.Conv2d_int8(16, 40, kernel, lut, grad="lre", dx=t(np.ones(256), torch.float32),
                              dw=t(np.ones(256), torch.float32), bias=True, padding=pad).to(DEV)
    x = torch.randn(3, 16, 13, 11, device=DEV)
    if relu:
        x = torch.relu(x)
    layer.train()
    with torch.no_grad():
        layer(x)                               # one EMA update
    layer.eval()
    spy = GemmSpy(monkeypatch)
    y = layer(x).detach()
    assert spy.seen == [1 if relu else 0]
    with monkeypatch.context() as m:
        full_tables(m)
        y_full = layer(x).detach()
    assert spy.seen[1:] == [None]
    assert torch.equal(y, y_full)
    sx = np.float32(layer.scale_x.item())
    sw = layer.scale_w.cpu().numpy()
    want, ctx = O.conv_int8_forward(x.cpu().numpy(), layer.weight.detach().cpu().numpy(),
                                    layer.bias.detach().cpu().numpy(), lut.cpu().numpy(), sx,
                                    sw, (kernel, kernel), (1, 1), (pad, pad), (1, 1))
    assert np.max(np.abs(y.double().cpu().numpy() - want) - 1e-5 * ctx["yabs"]) <= 1e-4


def test_eval_flag_tolerates_negatives_that_round_to_zero(monkeypatch):
    """The derived flag is a property of the quantized values: x slightly
    below 0 (quantized to 0, index 128) keeps it set."""
    import approxtorch_amd as at
    lut = t(lut_of("asym"), torch.float32)
    layer = at.nn.Conv2d_int8(8, 32, 3, lut, grad="ste", padding=1).to(DEV).eval()
    layer.scale_x.fill_(0.5)
    x = torch.relu(torch.randn(2, 8, 9, 9, device=DEV))
    x[0, 0, 0, :5] = -0.2                    # -0.2 / 0.5 rounds to -0
    spy = GemmSpy(monkeypatch)
    y = layer(x).detach()
    with monkeypatch.context() as m:
        full_tables(m)
        y_full = layer(x).detach()
    assert spy.seen == [1, None] and torch.equal(y, y_full)


@pytest.mark.parametrize("scale", [0.0, -3.0])
def test_training_flag_with_zero_or_negative_scale(scale, monkeypatch):
    """The statistic's x >= 0 flag stays a valid promise when scale_x holds 0
    or a negative value: the fake-quant divides by max(scale, 1e-12), so every
    quantized x is still >= 0; upper-table output equals full-table output."""
    import approxtorch_amd as at
    torch.manual_seed(17)
    lut = t(lut_of("perturbed"), torch.float32)
    layer = at.nn.Conv2d_int8(16, 32, 3, lut, grad="ste", bias=True, padding=1).to(DEV)
    layer.train()
    layer.scale_momentum = 0.0               # the EMA keeps scale_x as set
    layer.scale_x.fill_(scale)
    x = torch.relu(torch.randn(2, 16, 10, 10, device=DEV))
    spy = GemmSpy(monkeypatch)
    y = layer(x).detach()
    assert layer.scale_x.item() == scale and spy.seen == [1]
    with monkeypatch.context() as m:
        full_tables(m)
        y_full = _full_table_forward(layer, x, 3)
    assert torch.equal(y, y_full)


@pytest.mark.parametrize("xdtype", ["uint8", "float32"])
@pytest.mark.parametrize("upper", [True, False])
def test_bgemm_fake_int8_derives_the_flag(xdtype, upper, monkeypatch):
    """bgemm_fake_int8_forward_cuda_claude: the pack kernel derives the flag
    (set when every index >= 128) and the sums stay exact either way."""
    N, K, Lc, Oc = 2, 301, 700, 70
    r = gen(zlib.crc32(repr(("bgemm-flag", xdtype, upper)).encode()))
    xi = r.integers(128, 256, (N, K, Lc), dtype=np.uint8)
    if not upper:
        xi[1, 7, 9] = 127
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = lut_of("perturbed")
    xa = xi if xdtype == "uint8" else xi.astype(np.float32) - 128
    spy = GemmSpy(monkeypatch)
    y = ops.bgemm_fake_int8_claude(t(xa), t(wi.astype(np.float32) - 128), t(lut, torch.float32))
    assert spy.seen == [1 if upper else 0]
    assert np.array_equal(y.cpu().numpy().astype(np.int64), O.lut_gemm_i64(xi, wi, lut))


@pytest.mark.parametrize("upper", [True, False])
def test_gemm2d_derives_the_flag(upper, monkeypatch):
    """gemm_fake_int8_claude (torch.mm layout, strided pack): same flag."""
    M, K, Nn = 300, 129, 2600                # rows = N: B^T is the row operand
    r = gen(zlib.crc32(repr(("gemm2d-flag", upper)).encode()))
    a = r.integers(-128, 128, (M, K)).astype(np.float32)
    b = r.integers(0, 128, (K, Nn)).astype(np.float32)
    if not upper:
        b[5, 77] = -1
    lut = lut_of("asym")
    spy = GemmSpy(monkeypatch)
    y = ops.gemm_fake_int8_claude(t(a), t(b), t(lut, torch.float32)).cpu().numpy()
    assert spy.seen == [1 if upper else 0]
    ai = (a + 128).astype(np.uint8)
    bi = (b + 128).astype(np.uint8)
    want = O.lut_gemm_i64(ai.T[None], bi.T, lut)[0].T       # [M, N]
    assert np.array_equal(y.astype(np.int64), want)


@pytest.mark.parametrize("shape", [(2, 5, 7, 3), (3, 64, 10, 10)])
def test_fakequant_flags(shape):
    """atx_fakequant_fwd's nonneg and atx_fakequant_rows' upper flags: cleared
    exactly when some quantized value is negative; NaN (quantized to 0),
    negatives rounding to -0 and the operand's padding do not clear them."""
    r = gen(zlib.crc32(repr(("fq-flags", shape)).encode()))
    s = torch.full((), 0.25, device=DEV)
    x = np.abs(r.standard_normal(shape)).astype(np.float32)
    x.flat[3] = np.nan
    x.flat[5] = -0.1                         # -0.4 rounds to -0
    cases = [(x, 1)]
    xn = x.copy()
    xn.flat[-1] = -0.2                       # -0.8 rounds to -1
    cases.append((xn, 0))
    for xv, want in cases:
        f = ops.upper_flag(DEV)
        ops.fakequant_per_tensor(t(xv), s, -127, 127, want_q=False, q8_dtype=torch.int8,
                                 nonneg=f)
        assert int(f.item()) == want
        f = ops.upper_flag(DEV)
        ops.fakequant_rows(t(xv), s, -127, 127, 128, upper=f)
        assert int(f.item()) == want
