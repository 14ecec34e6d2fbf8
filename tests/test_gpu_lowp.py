"""fp16 / bf16 activations: the statistic and fake-quant kernels against the
reference's statements evaluated by torch on the GPU in that dtype (the
semantics the reference's unfused path has for a non-fp32 x,
nn/quantization.py:44-62, nn/Conv2d_int8.py:137-166), the oracle's
restatement of them (pinned here against those same statements), and
Conv2d_int8 layers fed such inputs against the oracle."""
import numpy as np
import pytest
import torch

import approxtorch_amd as at
from approxtorch_amd.backend import _lib as L
from approxtorch_amd.backend import ops
from approxtorch_amd.nn import quantization as Q
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16}


def sample(dt, n, seed, scale=3.0):
    """Values of dtype dt: normal draws, ties of x / s around the quantization
    grid, clipping magnitudes, zeros of both signs."""
    r = np.random.default_rng(seed)
    v = np.concatenate([r.standard_normal(n) * scale,
                        (np.arange(-300, 301) + 0.5) * 0.0371,
                        np.array([0.0, -0.0, 1e4, -1e4, 5.0, -5.0])]).astype(np.float32)
    return torch.from_numpy(v).to(DTYPES[dt]).to(DEV)


def torch_fakequant(x, scale, qmin, qmax, zero=None):
    # nn/quantization.py:44-52 / 72-80, the unfused statements
    s = torch.clamp(scale, min=1e-12)
    v = x / s if zero is None else x / s + zero
    mask = (v >= qmin) & (v <= qmax)
    return torch.clamp(torch.round(v), qmin, qmax), mask


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_fakequant_matches_torch_statements(dt, asym):
    """q (in the dtype), mask and the byte image bit for bit: kernel ==
    torch's statements on the GPU == oracle.fakequant_lowp."""
    x = sample(dt, 40000, 1)
    scale = torch.tensor(0.0371, device=DEV)
    zero = torch.tensor(3.0, device=DEV) if asym else None
    qmin, qmax = (0, 255) if asym else (-127, 127)
    want_q, want_m = torch_fakequant(x, scale, qmin, qmax, zero)
    assert want_q.dtype == x.dtype
    q, m, q8 = ops.fakequant_per_tensor(x, scale, qmin, qmax, zero_point=zero,
                                        q8_dtype=torch.uint8 if asym else torch.int8)
    assert q.dtype == x.dtype
    assert torch.equal(q, want_q) and torch.equal(m, want_m)
    assert torch.equal(q8.to(torch.int32), want_q.to(torch.int32))
    oq, om = O.fakequant_lowp(x.float().cpu().numpy(), np.float32(0.0371), qmin, qmax, dt,
                              zero=None if zero is None else np.float32(3.0))
    assert np.array_equal(oq, want_q.float().cpu().numpy())
    assert np.array_equal(om, want_m.cpu().numpy())
    # the fp32 kernel on the same values quantizes some of them differently
    q32, _, _ = ops.fakequant_per_tensor(x.float(), scale, qmin, qmax, zero_point=zero)
    assert not torch.equal(q32, q.float())


@pytest.mark.parametrize("go_fp32", [False, True])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_fakequant_backward_matches_torch_statements(dt, go_fp32):
    """grad_output * mask.to(dtype) / s (nn/quantization.py:58-62) with the
    gradient in the dtype, or in fp32 as autograd then casts it."""
    x = sample(dt, 20000, 2)
    scale = torch.tensor(0.0371, device=DEV)
    _, m = torch_fakequant(x, scale, -127, 127)
    r = np.random.default_rng(3)
    go32 = torch.from_numpy((r.standard_normal(x.numel()) * 2).astype(np.float32)).to(DEV)
    go = go32 if go_fp32 else go32.to(x.dtype)
    s = torch.clamp(scale, min=1e-12)
    want = go.to(x.dtype) * m.to(x.dtype) / s
    got = ops.fakequant_per_tensor_backward(go, m, scale, dtype=x.dtype)
    assert got.dtype == x.dtype and torch.equal(got, want)
    o = O.fakequant_lowp_backward(go.float().cpu().numpy(), m.cpu().numpy(),
                                  np.float32(0.0371), dt)
    assert np.array_equal(o, want.float().cpu().numpy())


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_statistics_match_torch_statements(dt):
    """scale_x <- m * (abs_max / 127) + (1 - m) * scale_x and the per-channel
    weight EMA / reset (nn/Conv2d_int8.py:137-166) run by torch on a tensor
    of the dtype, against the dtype-aware kernels and the oracle."""
    from approxtorch_amd.nn.Conv2d_int8 import _ema_coeffs
    tdt = DTYPES[dt]
    m = 0.05
    m32, om32 = _ema_coeffs(m)
    ws = ops._reduce_ws(torch.device(DEV))
    for seed in range(12):
        x = sample(dt, 3001 + seed, 10 + seed, scale=1.0 + seed)
        old = torch.tensor(0.0371, device=DEV)
        want = m * (x.abs().max() / ((127 - -127) / 2)) + (1 - m) * old
        assert want.dtype == torch.float32
        st = L.stream_of(x)
        sc, stat = old.clone(), torch.empty((), device=DEV)
        upper = torch.empty((), dtype=torch.int32, device=DEV)
        L.call("atx_absmax_ema_upper_dt", L.ptr(x), ops.dtype_code(x), x.numel(), L.ptr(ws),
               L.ptr(stat), 127.0, m32, om32, L.ptr(sc), L.ptr(upper), st)
        assert sc.item() == want.item() and upper.item() == int(bool((x >= 0).all()))
        assert stat.item() == x.abs().max().item()
        sc2, stat2 = old.clone(), torch.empty((), device=DEV)
        L.call("atx_absmax_dt", L.ptr(x), ops.dtype_code(x), x.numel(), L.ptr(ws),
               L.ptr(stat2), st)
        L.call("atx_ema_absmax_apply_dt", L.ptr(stat2), ops.dtype_code(x), 127.0, m32, om32,
               L.ptr(sc2), st)
        assert sc2.item() == want.item()
        assert want.item() == O.ema_absmax_lowp(x.float().cpu().numpy(), np.float32(0.0371),
                                                m, dt)
    r = np.random.default_rng(4)
    w = torch.from_numpy((r.standard_normal((37, 3, 3, 3)) * 0.1).astype(np.float32))
    w[6] = 0
    w = w.to(tdt).to(DEV)
    sw = torch.from_numpy((r.random(37) * 0.01).astype(np.float32)).to(DEV)
    for bits in (4, 8):
        qmax_w = 2 ** (bits - 1) - 1
        absmax = w.abs().amax(dim=(1, 2, 3))
        cur = torch.where(absmax > 0, absmax / qmax_w, sw)
        want = m * cur + (1 - m) * sw
        want_reset = torch.where(absmax > 0, absmax / qmax_w, torch.ones_like(absmax)).float()
        got = sw.clone()
        L.call("atx_weight_scale_ema_dt", L.ptr(w), ops.dtype_code(w), 37, 27, float(qmax_w),
               m32, om32, 0, L.ptr(got), L.stream_of(w))
        assert torch.equal(got, want)
        L.call("atx_weight_scale_ema_dt", L.ptr(w), ops.dtype_code(w), 37, 27, float(qmax_w),
               1.0, 0.0, 1, L.ptr(got), L.stream_of(w))
        assert torch.equal(got, want_reset)
        wn = w.float().cpu().numpy()
        assert np.array_equal(O.weight_scale_ema_lowp(wn, sw.cpu().numpy(), m, qmax_w, dt),
                              want.cpu().numpy())
        assert np.array_equal(O.weight_scale_ema_lowp(wn, None, m, qmax_w, dt, reset=True),
                              want_reset.cpu().numpy())


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_static_quantize_api(dt):
    """The public fake-quant functions: a 0-dim scale keeps x's dtype, a
    1-element or per-channel scale promotes to fp32 (torch's type promotion
    of the reference's statements), with their gradients."""
    x = sample(dt, 5000, 5)[:5000].reshape(1000, 5).contiguous()
    scale = torch.tensor(0.0371, device=DEV)
    xr = x.clone().requires_grad_()
    q = Q.static_quantize_int8(xr, scale)
    want, m = torch_fakequant(x, scale, -127, 127)
    assert q.dtype == x.dtype and torch.equal(q, want)
    go = torch.randn(q.shape, device=DEV).to(x.dtype)
    q.backward(go)
    assert xr.grad.dtype == x.dtype
    assert torch.equal(xr.grad, go * m.to(x.dtype) / torch.clamp(scale, min=1e-12))
    s1 = scale.view(1)
    q1 = Q.static_quantize_int8(x, s1)
    w1, _ = torch_fakequant(x, s1, -127, 127)
    assert q1.dtype == torch.float32 and w1.dtype == torch.float32 and torch.equal(q1, w1)
    sc = torch.rand(5, device=DEV) * 0.05 + 0.01
    qc = Q.static_quantize_int8(x, sc, ch_axis=1)
    wc, _ = torch_fakequant(x, sc.view(1, 5), -127, 127)
    assert qc.dtype == torch.float32 and torch.equal(qc, wc)
    zp = torch.tensor(7.0, device=DEV)
    qu = Q.static_quantize_uint8(x, scale, zp)
    wu, _ = torch_fakequant(x, scale, 0, 255, zp)
    assert qu.dtype == x.dtype and torch.equal(qu, wu)


def lut_perturbed(seed):
    r = np.random.default_rng(seed)
    a = np.arange(256) - 128
    p = a[:, None] * a[None, :]
    e = np.rint(r.normal(0, 1, p.shape) * (0.02 * np.abs(p) + 1))
    return np.clip(p + e, -32768, 32767).astype(np.float32).reshape(-1)


def close(got, want, absref, rtol=1e-5, atol=1e-4):
    got = got.detach().double().cpu().numpy()
    want = np.asarray(want, dtype=np.float64)
    excess = np.abs(got - want) - (atol + rtol * np.asarray(absref, dtype=np.float64))
    assert excess.max() <= 0, f"max excess {excess.max():.3g}"


def close_lowp(got, want, absref, scale, dt):
    """gx in the dtype: the GPU's fp32 gradient of the quantized x differs
    from the oracle's fp64 one by the fp32 evaluation bound (rel 1e-5 of the
    sum of |terms|, + 1e-4) before the STE divides by s and rounds to the
    dtype; allow that, divided by s, plus one unit in the last place of the
    dtype (2^-10 / 2^-7 relative)."""
    ulp = 2.0 ** (-10 if dt == "f16" else -7)
    got = got.detach().double().cpu().numpy()
    want = np.asarray(want, dtype=np.float64)
    tol = (1e-4 + 1e-5 * np.asarray(absref, dtype=np.float64)) + ulp * np.abs(want) + 1e-30
    assert (np.abs(got - want) <= tol).all(), f"max err {np.abs(got - want).max():.3g}"


@pytest.mark.parametrize("kind", ["ste", "lre", "custom"])
@pytest.mark.parametrize("geom", [(3, 1, 1), (1, 1, 0), (3, 2, 1)])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_conv2d_int8_lowp_input(dt, geom, kind):
    """Conv2d_int8 fed an fp16 / bf16 x in training mode (fp32 weights): the
    EMA scale as torch computes it for that dtype, y (fp32) against the
    oracle layer with the dtype's fake-quant, gx in the dtype, gw / gb fp32.
    custom: the pair-table estimator with DATE tables (the unfused path:
    static fake-quant in the dtype, then the conv Function)."""
    k, st, p = geom
    torch.manual_seed(7)
    lut = lut_perturbed(3)
    if kind == "ste":
        dx, dw = None, None
    elif kind == "lre":
        dx, dw = O.lre_tables(lut, "int8")
    else:
        dx, dw = (t.reshape(-1) for t in O.date_tables(lut.reshape(256, 256), 2))
    layer = at.nn.Conv2d_int8(6, 20, k, torch.from_numpy(lut).to(DEV), grad=kind,
                              dx=None if dx is None else torch.from_numpy(dx).to(DEV),
                              dw=None if dw is None else torch.from_numpy(dw).to(DEV),
                              bias=True, stride=st, padding=p, scale_momentum=0.5).to(DEV)
    layer.train()
    x = (torch.randn(3, 6, 11, 10, device=DEV) * 2).to(DTYPES[dt])
    sx0 = np.float32(layer.scale_x.item())
    sw0 = layer.scale_w.cpu().numpy()
    xr = x.clone().requires_grad_()
    y = layer(xr)
    assert y.dtype == torch.float32
    xn = x.float().cpu().numpy()
    sx = O.ema_absmax_lowp(xn, sx0, 0.5, dt)
    assert np.float32(layer.scale_x.item()) == sx
    w = layer.weight.detach().cpu().numpy()
    sw = O.weight_scale_ema(w, sw0, 0.5, 127)
    assert np.array_equal(layer.scale_w.cpu().numpy(), sw)
    k2, s2, p2, d2 = (k, k), (st, st), (p, p), (1, 1)
    want, ctx = O.conv_int8_forward(xn, w, layer.bias.detach().cpu().numpy(), lut, sx, sw,
                                    k2, s2, p2, d2, x_dtype=dt)
    close(y, want, ctx["yabs"])
    go = torch.randn_like(y)
    y.backward(go)
    tb = None if kind == "ste" else (dx, dw)
    gon = go.cpu().numpy()
    gx, gw, gb = O.conv_int8_backward(gon, ctx, sx, sw, kind, tb, k2, s2, p2, d2, x_dtype=dt)
    ax, aw, ab = O.conv_int8_backward(gon, ctx, sx, sw, kind, tb, k2, s2, p2, d2, absolute=True)
    assert xr.grad.dtype == x.dtype
    close_lowp(xr.grad, gx, ax * max(float(sx), 1e-12), sx, dt)
    close(layer.weight.grad, gw, aw)
    close(layer.bias.grad, gb, ab)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_conv2d_int8_half_module(dt):
    """A module converted to fp16 / bf16 (weights and bias of the dtype, as
    after model.half()): weight scales from the dtype-aware statistic,
    weight and bias gradients of the parameters' dtype (autograd casts the
    fp32 gradients, as for the reference), forward against the oracle."""
    tdt = DTYPES[dt]
    torch.manual_seed(8)
    lut = lut_perturbed(4)
    layer = at.nn.Conv2d_int8(5, 12, 3, torch.from_numpy(lut).to(DEV), grad="ste", bias=True,
                              padding=1, scale_momentum=1.0).to(DEV)
    with torch.no_grad():
        layer.weight.copy_(layer.weight.to(tdt).float())
    layer.weight.data = layer.weight.data.to(tdt)
    layer.bias.data = layer.bias.data.to(tdt)
    layer.train()
    sw0 = layer.scale_w.cpu().numpy()
    x = torch.randn(2, 5, 9, 9, device=DEV).to(tdt)
    y = layer(x)
    wn = layer.weight.detach().float().cpu().numpy()
    sw = O.weight_scale_ema_lowp(wn, sw0, 1.0, 127, dt)
    assert np.array_equal(layer.scale_w.cpu().numpy(), sw)
    sx = np.float32(layer.scale_x.item())
    want, ctx = O.conv_int8_forward(x.float().cpu().numpy(), wn,
                                    layer.bias.detach().float().cpu().numpy(), lut, sx, sw,
                                    (3, 3), (1, 1), (1, 1), (1, 1), x_dtype=dt)
    close(y, want, ctx["yabs"])
    y.backward(torch.randn_like(y))
    assert layer.weight.grad.dtype == tdt and layer.bias.grad.dtype == tdt
