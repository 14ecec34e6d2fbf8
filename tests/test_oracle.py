"""Pins the CPU oracle (oracle/oracle.py, oracle/lut_oracle.c) with checks that
do not restate its formulas: brute-force loops, closed forms, invariants and
library routines (torch on the CPU, scipy.stats.linregress)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O

rng = np.random.default_rng(1234)


def asym_lut():
    # test_naive_lut_ops.py:57-59 recipe: distinguishes lut[x][w] from lut[w][x]
    r = np.arange(256)[:, None]
    c = np.arange(256)[None, :]
    return (37 * r - 19 * c + 11).reshape(-1)


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (2, 5, 7, 3), (3, 33, 9, 17)])
def test_lut_gemm_matches_bruteforce_asymmetric_lut(shape):
    N, K, L, Oc = shape
    xi = rng.integers(0, 256, (N, K, L), dtype=np.uint8)
    wi = rng.integers(0, 256, (Oc, K), dtype=np.uint8)
    lut = asym_lut()
    y = O.lut_gemm_i64(xi, wi, lut)
    assert np.array_equal(y, O.lut_gemm_bruteforce(xi, wi, lut).astype(np.int64))
    # swapping the operand roles must change the result for this LUT
    lut_t = lut.reshape(256, 256).T.reshape(-1)
    if K > 1:
        assert not np.array_equal(y, O.lut_gemm_i64(xi, wi, lut_t))


def test_exact_product_lut_is_integer_gemm():
    a = np.arange(256) - 128
    lut = (a[:, None] * a[None, :]).reshape(-1)
    xi = rng.integers(0, 256, (4, 37, 21), dtype=np.uint8)
    wi = rng.integers(0, 256, (11, 37), dtype=np.uint8)
    want = np.einsum("nkl,ok->nol", xi.astype(np.int64) - 128, wi.astype(np.int64) - 128)
    assert np.array_equal(O.lut_gemm_i64(xi, wi, lut), want)


def test_linearity_in_the_lut():
    xi = rng.integers(0, 256, (2, 19, 13), dtype=np.uint8)
    wi = rng.integers(0, 256, (5, 19), dtype=np.uint8)
    p = rng.integers(-300, 300, 65536)
    q = rng.integers(-300, 300, 65536)
    lhs = O.lut_gemm_i64(xi, wi, 3 * p - 7 * q)
    rhs = 3 * O.lut_gemm_i64(xi, wi, p) - 7 * O.lut_gemm_i64(xi, wi, q)
    assert np.array_equal(lhs, rhs)


def test_f32_sum_exact_for_small_integers_and_sequential_for_halves():
    xi = rng.integers(0, 256, (2, 40, 9), dtype=np.uint8)
    wi = rng.integers(0, 256, (3, 40), dtype=np.uint8)
    lut = rng.integers(-1000, 1000, 65536)
    assert np.array_equal(O.lut_gemm_f32(xi, wi, lut.astype(np.float32)),
                          O.lut_gemm_i64(xi, wi, lut).astype(np.float32))
    half = (rng.integers(-2000, 2000, 65536) / 2 + 1e-3).astype(np.float32)
    got = O.lut_gemm_f32(xi[:1, :, :2], wi[:1], half)
    for l in range(2):
        acc = np.float32(0)
        for k in range(40):
            acc = np.float32(acc + half[int(xi[0, k, l]) * 256 + int(wi[0, k])])
        assert got[0, 0, l] == acc


def test_lut_class_boundaries():
    base = np.zeros(65536, dtype=np.float32)
    t = base.copy(); t[5] = 32767; t[6] = -32767
    assert O.lut_class(t) == 0
    t = base.copy(); t[5] = 32768
    assert O.lut_class(t) == 1
    t = base.copy(); t[5] = 65535
    assert O.lut_class(t) == 1
    t = base.copy(); t[5] = 65536
    assert O.lut_class(t) == 2
    t = base.copy(); t[5] = 32768; t[6] = -1
    assert O.lut_class(t) == 2
    t = base.copy(); t[5] = 0.5
    assert O.lut_class(t) == 2


@pytest.mark.parametrize("geom", [((3, 3), (1, 1), (1, 1), (1, 1)), ((7, 7), (2, 2), (3, 3), (1, 1)),
                                  ((3, 3), (2, 1), (0, 2), (2, 1)), ((1, 1), (2, 2), (0, 0), (1, 1))])
def test_unfold_and_fold_match_torch(geom):
    k, s, p, d = geom
    x = rng.standard_normal((2, 3, 11, 9))
    ref = F.unfold(torch.from_numpy(x), k, dilation=d, padding=p, stride=s).numpy()
    assert np.allclose(O.unfold_values(x, k, s, p, d, 0.0), ref)
    OH, OW = O.out_size(11, 9, k, s, p, d)
    col = rng.standard_normal((2, 3 * k[0] * k[1], OH * OW))
    ref_f = F.fold(torch.from_numpy(col), (11, 9), k, dilation=d, padding=p, stride=s).numpy()
    assert np.allclose(O.fold(col, (2, 3, 11, 9), k, s, p, d), ref_f)


def test_im2col_index_padding_and_order():
    img = rng.integers(-128, 128, (2, 3, 5, 6)).astype(np.int8)
    k, s, p, d = (3, 2), (2, 1), (1, 2), (1, 2)
    got = O.im2col_index(O.image_index(img), k, s, p, d, 128)
    vals = O.unfold_values(img.astype(np.float64) + 128, k, s, p, d, 128.0)
    assert np.array_equal(got.astype(np.float64), vals)


def test_fakequant_matches_reference_formula_in_torch():
    # nn/quantization.py:48-52, evaluated with torch on the CPU
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 3,
                        np.array([0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 127.4, 127.6, -127.5, -200,
                                  np.nan, 0.0, -0.0], dtype=np.float32)])
    for scale in (np.float32(0.023), np.float32(1.0), np.float32(0.0)):
        q, m = O.fakequant(x, scale, -127, 127)
        xt = torch.from_numpy(x)
        s = torch.clamp(torch.tensor(scale), min=1e-12)
        v = xt / s
        assert np.array_equal(m, ((v >= -127) & (v <= 127)).numpy())
        qt = torch.clamp(torch.round(v), -127, 127).numpy()
        assert np.array_equal(q, qt, equal_nan=True)
    # asymmetric: v = x/s + z
    z = np.float32(17)
    q, m = O.fakequant(x, np.float32(0.05), 0, 255, zero=z)
    v = torch.from_numpy(x) / torch.tensor(np.float32(0.05)) + torch.tensor(z)
    assert np.array_equal(q, torch.clamp(torch.round(v), 0, 255).numpy(), equal_nan=True)
    assert np.array_equal(m, ((v >= 0) & (v <= 255)).numpy())


def test_fakequant_hand_cases():
    q, m = O.fakequant(np.array([0.5, 1.5, 2.5, 130.0, -130.0], dtype=np.float32),
                       np.float32(1.0), -127, 127)
    assert q.tolist() == [0.0, 2.0, 2.0, 127.0, -127.0]
    assert m.tolist() == [True, True, True, False, False]
    g = O.fakequant_backward(np.array([1, 1, 1, 1, 1], dtype=np.float32), m, np.float32(0.5))
    assert g.tolist() == [2.0, 2.0, 2.0, 0.0, 0.0]


def gpu_div(t, number):
    """`t / number` (number a python scalar) as torch evaluates it on the GPU,
    where the reference runs: t times the fp32 reciprocal of the number (its
    true-divide kernel's host-scalar path).  The CPU kernel divides exactly,
    so the reference statements below are evaluated on the CPU with this
    substitution; test_gpu_ops.py's
    test_torch_gpu_divides_by_numbers_via_the_reciprocal checks the device
    behaviour itself."""
    return t * torch.tensor(np.float32(1) / np.float32(number))


def test_div_by_number_is_the_reciprocal_product():
    """oracle.div_by_number differs from exact fp32 division for some values
    (so the choice matters) and equals v * fl(1/n) for every one."""
    v = (rng.random(20000) * 100).astype(np.float32)
    got = O.div_by_number(v, 127.0)
    assert np.array_equal(got, gpu_div(torch.from_numpy(v), 127.0).numpy())
    assert (got != (v / np.float32(127))).sum() > 100


def test_ema_and_qparams_match_torch_bitwise():
    for m in (0.05, 0.1, 0.3333):
        x = rng.standard_normal(777).astype(np.float32) * 4
        old = np.float32(0.0371)
        xt = torch.from_numpy(x)
        cur = gpu_div(xt.abs().max(), (127 - -127) / 2)
        want = (m * cur + (1 - m) * torch.tensor(old)).item()
        assert O.ema_absmax(x, old, m) == np.float32(want)
        w = rng.standard_normal((6, 3, 3, 3)).astype(np.float32)
        w[2] = 0
        sw = rng.random(6).astype(np.float32)
        wt = torch.from_numpy(w)
        absmax = wt.abs().amax(dim=(1, 2, 3))
        cur_w = torch.where(absmax > 0, gpu_div(absmax, 7), torch.from_numpy(sw))
        want_w = (m * cur_w + (1 - m) * torch.from_numpy(sw)).numpy()
        assert np.array_equal(O.weight_scale_ema(w, sw, m, 7), want_w)
    mn = torch.tensor([-1.3, 0.4, -0.0, -5.0])
    mx = torch.tensor([2.2, 3.0, 0.0, -1.0])
    mnc, mxc = torch.clamp(mn, max=0.0), torch.clamp(mx, min=0.0)
    sc = torch.clamp(gpu_div(mxc - mnc, 255), min=1e-12)
    zr = torch.round(-mnc / sc).clamp(0.0, 255.0)
    s, z = O.uint8_qparams(mn.numpy(), mx.numpy())
    assert np.array_equal(s, sc.numpy()) and np.array_equal(z, zr.numpy())


def _torch_qparams(mn, mx, qmax):
    # nn/Conv2d_uint8.py:11-23, evaluated by torch
    mn = torch.clamp(mn, max=0.0)
    mx = torch.clamp(mx, min=0.0)
    scale = torch.clamp(gpu_div(mx - mn, qmax), min=1e-12)
    return scale, torch.round(-mn / scale).clamp(0.0, float(qmax))


@pytest.mark.parametrize("m", [0.05, 0.1, 0.3333])
def test_ema_minmax_matches_reference_torch_expression(m):
    """oracle.ema_minmax against the reference's own torch statements
    (nn/Conv2d_uint8.py:225-240): amin/amax, `m * mn + (1 - m) * x_min`,
    then uint8_qparams -- bitwise, including a range that excludes 0."""
    for shift in (0.0, 3.0, -3.0):
        x = (rng.standard_normal(1031).astype(np.float32) * 2 + shift).astype(np.float32)
        xmin, xmax = np.float32(-0.731), np.float32(1.913)
        xt = torch.from_numpy(x)
        tmin = m * xt.amin() + (1 - m) * torch.tensor(xmin)
        tmax = m * xt.amax() + (1 - m) * torch.tensor(xmax)
        ts, tz = _torch_qparams(tmin, tmax, 255)
        nmin, nmax, s, z = O.ema_minmax(x, xmin, xmax, m)
        assert nmin == tmin.item() and nmax == tmax.item()
        assert s == ts.item() and z == tz.item()


@pytest.mark.parametrize("qmax", [255, 15])
def test_weight_minmax_ema_matches_reference_torch_expression(qmax):
    """oracle.weight_minmax_ema against nn/Conv2d_uint8.py:242-255 evaluated
    by torch (per-channel amin/amax over dims 1.., the same EMA, qparams)."""
    w = rng.standard_normal((7, 4, 3, 3)).astype(np.float32)
    w[3] = np.abs(w[3])            # a channel with min > 0
    w[5] = -np.abs(w[5])           # a channel with max < 0
    w[6] = 0
    wmin = rng.standard_normal(7).astype(np.float32)
    wmax = np.abs(rng.standard_normal(7)).astype(np.float32)
    m = 0.1
    wt = torch.from_numpy(w)
    tmin = m * wt.amin(dim=(1, 2, 3)) + (1 - m) * torch.from_numpy(wmin)
    tmax = m * wt.amax(dim=(1, 2, 3)) + (1 - m) * torch.from_numpy(wmax)
    ts, tz = _torch_qparams(tmin, tmax, qmax)
    a, b, s, z = O.weight_minmax_ema(w, wmin, wmax, m, qmax)
    for got, want in ((a, tmin), (b, tmax), (s, ts), (z, tz)):
        assert np.array_equal(got, want.numpy())


@pytest.mark.parametrize("bits", [3, 4, 8])
def test_weight_scale_reset_matches_reference_torch_expression(bits):
    """oracle.weight_scale_reset against nn/Conv2d_int8.py:160-167 in torch:
    where(absmax > 0, absmax / qmax_w, 1), zero channels reset to 1."""
    w = rng.standard_normal((6, 5, 3, 3)).astype(np.float32)
    w[1] = 0
    qmax_w = 2 ** (bits - 1) - 1
    absmax = torch.from_numpy(w).abs().amax(dim=(1, 2, 3))
    want = torch.where(absmax > 0, gpu_div(absmax, qmax_w), torch.ones_like(absmax))
    got = O.weight_scale_reset(w, qmax_w)
    assert np.array_equal(got, want.numpy())
    assert got[1] == 1.0


def test_quant_index_matches_torch_round_and_clamp():
    """quant_index = clamp(round-half-even(v) + offset, 0, 255), the index of
    csrc/claude/bgemm_lut_kernels.cuh:62-67, checked against torch.round /
    clamp (half-even ties, both clip edges, large magnitudes)."""
    v = np.concatenate([np.arange(-140, 141, 0.5, dtype=np.float32),
                        np.array([-1e9, 1e9, -0.5, 0.5, 1.5, 2.5, -2.5, 127.5, -128.5],
                                 dtype=np.float32),
                        rng.uniform(-300, 300, 2000).astype(np.float32)])
    for offset in (128, 0):
        want = (torch.round(torch.from_numpy(v)).clamp(-1024, 1024) + offset).clamp(0, 255)
        assert np.array_equal(O.quant_index(v, offset), want.to(torch.uint8).numpy())
    # NaN maps to the quantized zero (documented choice: the reference's
    # float->int conversion of NaN is unspecified)
    assert O.quant_index(np.array([np.nan], dtype=np.float32), 128)[0] == 128


def test_lut_map_and_pad_match_torch_take_and_pad():
    """lut_map = table.take(idx) and lut_map_pad = F.pad(table[idx], value =
    table[128]) (csrc/claude/bgemm_lre_backward_claude.cu:95-127,276-307)."""
    table = rng.standard_normal(256).astype(np.float32)
    idx = rng.integers(0, 256, (2, 3, 5, 7)).astype(np.uint8)
    tt, it = torch.from_numpy(table), torch.from_numpy(idx.astype(np.int64))
    assert np.array_equal(O.lut_map(idx, table), tt.take(it).numpy())
    for p in ((1, 1), (0, 2), (3, 0)):
        want = F.pad(tt.take(it), (p[1], p[1], p[0], p[0]), value=float(table[128]))
        assert np.array_equal(O.lut_map_pad(idx, table, p), want.numpy())


def test_custom_grads_match_bruteforce_loops():
    """The C pair-table gradients (lut_oracle.c) against explicit loops over
    the definition (csrc/naive_cuda/bgemm_custom_grad_naive.cu:28-92) with a
    non-separable table, which catches swapped table indices or operands."""
    N, K, L, Oc = 2, 3, 5, 4
    xi = rng.integers(0, 256, (N, K, L)).astype(np.uint8)
    wi = rng.integers(0, 256, (Oc, K)).astype(np.uint8)
    go = rng.standard_normal((N, Oc, L))
    dxl = rng.standard_normal((256, 256))
    dwl = rng.standard_normal((256, 256))
    gx, gw = O.gemm_grads(go, xi, wi, "custom", (dxl, dwl))
    ax, aw = O.gemm_grads(go, xi, wi, "custom", (dxl, dwl), absolute=True)
    ex, ew = np.zeros((N, K, L)), np.zeros((Oc, K))
    bx, bw = np.zeros((N, K, L)), np.zeros((Oc, K))
    for n in range(N):
        for k in range(K):
            for l in range(L):
                for o in range(Oc):
                    a, b = int(xi[n, k, l]), int(wi[o, k])
                    ex[n, k, l] += go[n, o, l] * dxl[a, b]
                    ew[o, k] += go[n, o, l] * dwl[a, b]
                    bx[n, k, l] += abs(go[n, o, l] * dxl[a, b])
                    bw[o, k] += abs(go[n, o, l] * dwl[a, b])
    for got, want in ((gx, ex), (gw, ew), (ax, bx), (aw, bw)):
        assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_lre_tables_closed_form_and_linregress():
    a = np.arange(256) - 128
    ga, gb = O.lre_tables((a[:, None] * a[None, :]).astype(np.float32))
    assert np.allclose(ga, a) and np.allclose(gb, a)
    from scipy.stats import linregress
    lut = rng.integers(-2000, 2000, (256, 256)).astype(np.float32)
    ga, gb = O.lre_tables(lut)
    for y in (0, 77, 255):
        assert abs(ga[y] - linregress(a, lut[:, y]).slope) < 1e-5
        assert abs(gb[y] - linregress(a, lut[y, :]).slope) < 1e-5


def test_date_closed_forms():
    i = np.arange(256, dtype=np.float64)
    lin = (3 * i[:, None] + 5 * i[None, :]).astype(np.float32)
    ga, gb = O.date_tables(lin, 2)
    assert np.allclose(ga, 3) and np.allclose(gb, 5)
    quad = np.repeat((i * i)[:, None], 256, axis=1).astype(np.float32)
    ga, _ = O.date_tables(quad, 2)
    inner = np.arange(3, 253)
    assert np.allclose(ga[inner, 0], 2 * inner)           # d/da of a^2 = 2a
    assert np.allclose(ga[0, 0], (quad[255, 0] - quad[0, 0]) / 255)


def test_gemm_grads_estimators_agree_on_exact_tables():
    xi = rng.integers(0, 256, (2, 7, 5), dtype=np.uint8)
    wi = rng.integers(0, 256, (3, 7), dtype=np.uint8)
    go = rng.standard_normal((2, 3, 5))
    gx, gw = O.gemm_grads(go, xi, wi, "ste")
    want_x = np.einsum("nol,ok->nkl", go, wi.astype(np.float64) - 128)
    want_w = np.einsum("nol,nkl->ok", go, xi.astype(np.float64) - 128)
    assert np.allclose(gx, want_x) and np.allclose(gw, want_w)
    dec = np.arange(256, dtype=np.float32) - 128
    lx, lw = O.gemm_grads(go, xi, wi, "lre", (dec, dec))
    assert np.allclose(lx, gx) and np.allclose(lw, gw)
    a = np.arange(256) - 128.0
    dxl = np.repeat(a[None, :], 256, axis=0)       # d(x*w)/dx = w
    dwl = np.repeat(a[:, None], 256, axis=1)       # d(x*w)/dw = x
    cx, cw = O.gemm_grads(go, xi, wi, "custom", (dxl, dwl))
    assert np.allclose(cx, gx) and np.allclose(cw, gw)


def _geoms():
    return [((3, 3), (1, 1), (1, 1), (1, 1)), ((3, 3), (2, 2), (1, 1), (1, 1)),
            ((1, 1), (1, 1), (0, 0), (1, 1)), ((3, 1), (1, 2), (2, 0), (2, 1))]


@pytest.mark.parametrize("geom", _geoms())
def test_int8_layer_exact_lut_equals_float_conv(geom):
    k, s, p, d = geom
    x = rng.standard_normal((2, 4, 9, 8)).astype(np.float32)
    w = rng.standard_normal((5, 4, *k)).astype(np.float32) * 0.3
    b = rng.standard_normal(5).astype(np.float32)
    sx = np.float32(np.abs(x).max() / 127)
    sw = (np.abs(w).reshape(5, -1).max(axis=1) / 127).astype(np.float32)
    a = np.arange(256) - 128
    lut = (a[:, None] * a[None, :]).reshape(-1)
    y, _ = O.conv_int8_forward(x, w, b, lut, sx, sw, k, s, p, d)
    qx, _ = O.fakequant(x, sx, -127, 127)
    qw, _ = O.fakequant(w, sw.reshape(5, 1, 1, 1), -127, 127)
    ref = F.conv2d(torch.from_numpy(qx).double(), torch.from_numpy(qw).double(), None, s, p, d)
    sc = (sx * sw).astype(np.float32).astype(np.float64)
    ref = ref.numpy() * sc[None, :, None, None] + b[None, :, None, None]
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("geom", _geoms())
def test_int8_layer_ste_grads_match_torch_autograd(geom):
    k, s, p, d = geom
    x = rng.standard_normal((2, 3, 8, 7)).astype(np.float32)
    w = rng.standard_normal((4, 3, *k)).astype(np.float32) * 0.3
    sx = np.float32(np.abs(x).max() / 100)     # some values clip
    sw = (np.abs(w).reshape(4, -1).max(axis=1) / 100).astype(np.float32)
    a = np.arange(256) - 128
    lut = ((a[:, None] * a[None, :]) >> 3).reshape(-1)
    go = rng.standard_normal((2, 4, *O.out_size(8, 7, k, s, p, d)))
    _, ctx = O.conv_int8_forward(x, w, None, lut, sx, sw, k, s, p, d)
    gx, gw, _ = O.conv_int8_backward(go, ctx, sx, sw, "ste", None, k, s, p, d)
    # the reference composition with torch autograd (STE = exact product)
    xt = torch.from_numpy(x).double().requires_grad_()
    wt = torch.from_numpy(w).double().requires_grad_()
    vx = xt / float(sx)
    mx = ((vx >= -127) & (vx <= 127)).double()
    qx = torch.clamp(torch.round(vx), -127, 127).detach() + (vx - vx.detach()) * mx
    vw = wt / torch.from_numpy(sw).double().view(-1, 1, 1, 1)
    mw = ((vw >= -127) & (vw <= 127)).double()
    qw = torch.clamp(torch.round(vw), -127, 127).detach() + (vw - vw.detach()) * mw
    y = F.conv2d(qx, qw, None, s, p, d)
    sc = torch.from_numpy((sx * sw).astype(np.float32)).double().view(1, -1, 1, 1)
    (y * sc * torch.from_numpy(go)).sum().backward()
    assert np.allclose(gx, xt.grad.numpy(), rtol=1e-9, atol=1e-9)
    assert np.allclose(gw, wt.grad.numpy(), rtol=1e-9, atol=1e-9)


def test_uint8_layer_exact_lut_is_centred_conv_and_grads_match_autograd():
    k, s, p, d = (3, 3), (1, 1), (1, 1), (1, 1)
    x = rng.standard_normal((2, 3, 7, 6)).astype(np.float32) + 0.3
    w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32) * 0.2
    sx, zx = O.uint8_qparams(x.min(), x.max())
    sw, zw = O.uint8_qparams(w.reshape(4, -1).min(1), w.reshape(4, -1).max(1))
    v = np.arange(256)
    lut = (v[:, None] * v[None, :]).reshape(-1)
    y, ctx = O.conv_uint8_forward(x, w, None, lut, sx, zx, sw, zw, k, s, p, d)
    qx, _ = O.fakequant(x, sx, 0, 255, zero=zx)
    qw, _ = O.fakequant(w, sw.reshape(4, 1, 1, 1), 0, 255, zero=zw.reshape(4, 1, 1, 1))
    cx = torch.from_numpy(qx).double() - float(zx)
    cw = torch.from_numpy(qw).double() - torch.from_numpy(zw).double().view(-1, 1, 1, 1)
    sc = (sx * sw).astype(np.float32).astype(np.float64)
    ref = F.conv2d(cx, cw, None, s, p, d).numpy() * sc[None, :, None, None]
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-9)
    # STE gradients vs torch autograd of the reference's unfold formulation
    go = rng.standard_normal(y.shape)
    gx, gw, _ = O.conv_uint8_backward(go, ctx, sx, sw, "ste", None, k, s, p, d)
    xt = torch.from_numpy(x).double().requires_grad_()
    wt = torch.from_numpy(w).double().requires_grad_()
    vx = xt / float(sx) + float(zx)
    mx = ((vx >= 0) & (vx <= 255)).double()
    q_x = torch.clamp(torch.round(vx), 0, 255).detach() + (vx - vx.detach()) * mx
    vw = wt / torch.from_numpy(sw).double().view(-1, 1, 1, 1) + \
        torch.from_numpy(zw).double().view(-1, 1, 1, 1)
    mw = ((vw >= 0) & (vw <= 255)).double()
    q_w = torch.clamp(torch.round(vw), 0, 255).detach() + (vw - vw.detach()) * mw
    xp = F.pad(q_x - float(zx), (1, 1, 1, 1)) + float(zx)
    xu = F.unfold(xp, k, dilation=d, padding=0, stride=s)
    wu = q_w.view(4, -1)
    lutsum = torch.einsum("nkl,ok->nol", xu, wu)
    corr = lutsum - torch.from_numpy(zw).double().view(1, -1, 1) * xu.sum(1, keepdim=True) \
        - (float(zx) * wu.sum(1)).view(1, -1, 1) + 27 * float(zx) * \
        torch.from_numpy(zw).double().view(1, -1, 1)
    yy = corr.view(go.shape) * torch.from_numpy(sc).view(1, -1, 1, 1)
    (yy * torch.from_numpy(go)).sum().backward()
    assert np.allclose(gx, xt.grad.numpy(), rtol=1e-9, atol=1e-8)
    assert np.allclose(gw, wt.grad.numpy(), rtol=1e-9, atol=1e-8)


@pytest.mark.parametrize("geom", [((3, 3), (1, 1), (1, 1), (1, 1)), ((3, 3), (2, 2), (1, 1), (1, 1)),
                                  ((5, 3), (1, 2), (2, 0), (2, 1))])
def test_dwconv_oracle_bruteforce_and_ste_autograd(geom):
    """Depthwise oracle (per-channel LUT conv): the forward against a direct
    loop over pixels and taps with an asymmetric LUT (out-of-image taps = row
    128), the STE gradients of an exact-product LUT against torch's grouped
    conv2d autograd in fp64."""
    k, s, p, d = geom
    C = 3
    x = rng.standard_normal((2, C, 7, 6)).astype(np.float32)
    w = rng.standard_normal((C, 1, *k)).astype(np.float32) * 0.4
    b = rng.standard_normal(C).astype(np.float32)
    sx = np.float32(np.abs(x).max() / 100)
    sw = (np.abs(w).reshape(C, -1).max(axis=1) / 100).astype(np.float32)
    v = np.arange(256)
    lut = (37 * v[:, None] - 19 * v[None, :] + 11).reshape(-1)
    y, _ = O.dwconv_int8_forward(x, w, b, lut, sx, sw, k, s, p, d)
    qx, _ = O.fakequant(x, sx, -127, 127)
    qw, _ = O.fakequant(w, sw.reshape(C, 1, 1, 1), -127, 127)
    xi = O.image_index(qx, 128)
    wi = O.image_index(qw.reshape(C, -1), 128)
    OH, OW = O.out_size(7, 6, k, s, p, d)
    sc = (sx * sw).astype(np.float32).astype(np.float64)
    for n in range(2):
        for c in range(C):
            for oh in range(OH):
                for ow in range(OW):
                    acc = 0
                    for i in range(k[0]):
                        for j in range(k[1]):
                            ih, iw = oh * s[0] - p[0] + i * d[0], ow * s[1] - p[1] + j * d[1]
                            xv = int(xi[n, c, ih, iw]) if 0 <= ih < 7 and 0 <= iw < 6 else 128
                            acc += int(lut[xv * 256 + int(wi[c, i * k[1] + j])])
                    assert y[n, c, oh, ow] == acc * sc[c] + np.float64(b[c])
    a = v - 128
    plut = (a[:, None] * a[None, :]).reshape(-1)
    go = rng.standard_normal((2, C, OH, OW))
    _, ctxs = O.dwconv_int8_forward(x, w, None, plut, sx, sw, k, s, p, d)
    gx, gw, _ = O.dwconv_int8_backward(go, ctxs, sx, sw, "ste", None, k, s, p, d)
    xt = torch.from_numpy(x).double().requires_grad_()
    wt = torch.from_numpy(w).double().requires_grad_()
    vx = xt / float(sx)
    mx = ((vx >= -127) & (vx <= 127)).double()
    qxt = torch.clamp(torch.round(vx), -127, 127).detach() + (vx - vx.detach()) * mx
    vw = wt / torch.from_numpy(sw).double().view(-1, 1, 1, 1)
    mw = ((vw >= -127) & (vw <= 127)).double()
    qwt = torch.clamp(torch.round(vw), -127, 127).detach() + (vw - vw.detach()) * mw
    yt = F.conv2d(qxt, qwt, None, s, p, d, groups=C)
    sct = torch.from_numpy((sx * sw).astype(np.float32)).double().view(1, -1, 1, 1)
    (yt * sct * torch.from_numpy(go)).sum().backward()
    assert np.allclose(gx, xt.grad.numpy(), rtol=1e-9, atol=1e-9)
    assert np.allclose(gw, wt.grad.numpy(), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("h", [1, 2, 5, 32, 100])
def test_date_boundary_indices(h):
    """grad_lut.py:82-102 switches from the boundary fallback to the central
    difference strictly inside (h, 255 - h).  With LUT[a][b] = a^2 the
    smoothed line inside the window range is a^2 + h(h+1)/3, so the central
    difference is 2a there, while the fallback is (255^2 - 0) / 255 = 255
    (the raw ends).  Indices h, h+1, 254-h and 255-h tell the two apart, so
    an off-by-one in either bound fails; the same along b."""
    i = np.arange(256, dtype=np.float64)
    sq = (i * i).astype(np.float32)
    lut_a = np.repeat(sq[:, None], 256, axis=1)          # varies along a
    lut_b = np.repeat(sq[None, :], 256, axis=0)          # varies along b
    ga, _ = O.date_tables(lut_a, h)
    _, gb = O.date_tables(lut_b, h)
    for idx in (h, h + 1, 254 - h, 255 - h, 0, 255, 128):
        inside = h < idx < 255 - h
        want = 2.0 * idx if inside else 255.0
        assert np.allclose(ga[idx, :], want, rtol=1e-4), (h, idx, ga[idx, 0], want)
        assert np.allclose(gb[:, idx], want, rtol=1e-4), (h, idx, gb[0, idx], want)


def test_lre_table_roles_with_distinct_slopes():
    """grad_x reads dx at the weight index and grad_w reads dw at the
    activation index (NAIVE-README:222-232; grad_lut.py:14-37 fits grad_a per
    column, grad_b per row).  A LUT linear in x with a per-w slope c(w) plus a
    per-w offset makes grad_a = c exactly and the true d/dx of the sum
    sum_o go * c(w[o,k]); a LUT linear in w with slope e(x) gives grad_b = e
    and d/dw = sum go * e(x).  The slopes differ per index and between the two
    cases, so a swapped table or a swapped index fails."""
    r = np.random.default_rng(21)
    v = np.arange(256, dtype=np.float64) - 128
    c = r.integers(-9, 10, 256).astype(np.float64)
    e = r.integers(-9, 10, 256).astype(np.float64)
    off_w = r.integers(-50, 50, 256).astype(np.float64)
    off_x = r.integers(-50, 50, 256).astype(np.float64)
    lut_x = v[:, None] * c[None, :] + off_w[None, :]        # LUT[x][w], linear in x
    lut_w = v[None, :] * e[:, None] + off_x[:, None]        # linear in w
    ga, _ = O.lre_tables(lut_x.reshape(-1))
    _, gb = O.lre_tables(lut_w.reshape(-1))
    assert np.allclose(ga, c, atol=1e-5) and np.allclose(gb, e, atol=1e-5)
    xi = r.integers(0, 256, (2, 9, 5), dtype=np.uint8)
    wi = r.integers(0, 256, (4, 9), dtype=np.uint8)
    go = r.standard_normal((2, 4, 5))
    gx, _ = O.gemm_grads(go, xi, wi, "lre", (ga, np.zeros(256)))
    _, gw = O.gemm_grads(go, xi, wi, "lre", (np.zeros(256), gb))
    want_x = np.einsum("nol,ok->nkl", go, c[wi.astype(np.int64)])
    want_w = np.einsum("nol,nkl->ok", go, e[xi.astype(np.int64)])
    assert np.allclose(gx, want_x, atol=1e-9) and np.allclose(gw, want_w, atol=1e-9)
    # the roles swapped give something else
    sx, _ = O.gemm_grads(go, xi, wi, "lre", (gb, np.zeros(256)))
    assert not np.allclose(sx, want_x)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_round_to_matches_torch_conversion(dtype):
    """oracle.round_to against torch's fp32 -> fp16 / bf16 conversion (round
    to nearest even): ties at both parities, subnormals, overflow, inf, NaN."""
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    v = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10,
                        rng.standard_normal(2000).astype(np.float32) * 1e-6,
                        np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -8, 1 + 3 * 2 ** -8,
                                  65519.0, 65520.0, 3.4e38, -3.4e38, np.inf, -np.inf, 0.0,
                                  -0.0], np.float32)])
    want = torch.from_numpy(v).to(tdt).float().numpy()
    got = O.round_to(v, dtype)
    assert np.array_equal(got, want)
    assert np.isnan(O.round_to(np.array([np.nan], np.float32), dtype)).all()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_fakequant_lowp_differs_from_fp32_and_keeps_integers(dtype):
    """The dtype's rounding of s and of x / s changes some quantized values
    against the fp32 fake-quant of the same x (so the semantics matter), q
    is integer-valued and within [qmin, qmax], and the gradient is nonzero
    exactly on the mask."""
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    x = torch.from_numpy((rng.standard_normal(50000) * 3).astype(np.float32)).to(tdt).float()
    x = x.numpy()
    q, m = O.fakequant_lowp(x, np.float32(0.0371), -127, 127, dtype)
    q32, _ = O.fakequant(x, np.float32(0.0371), -127, 127)
    assert (q != q32).sum() > 0
    assert np.array_equal(q, np.rint(q)) and q.min() >= -127 and q.max() <= 127
    g = O.fakequant_lowp_backward(np.ones_like(x), m, np.float32(0.0371), dtype)
    assert np.all((g != 0) == m)
