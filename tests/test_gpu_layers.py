"""Layer-level GPU parity: Conv2d_int8 / Conv2d_uint8 forward and backward
(STE, LRE, custom) against the CPU oracle's restatement of the reference
layers; outputs and gradients within rel 1e-5 / abs 1e-4, the relative part
taken against the sum of |terms| of each value (the bound any fp32
evaluation order meets, including the reference's own)."""
import numpy as np
import pytest
import torch

import approxtorch_amd as at
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-5, 1e-4


def close(got, want, absref):
    got = got.detach().double().cpu().numpy()
    want = np.asarray(want, dtype=np.float64)
    excess = np.abs(got - want) - (ATOL + RTOL * np.asarray(absref, dtype=np.float64))
    assert excess.max() <= 0, \
        f"max excess {excess.max():.3g} at {np.unravel_index(excess.argmax(), want.shape)}"


def perturbed_lut(seed=0):
    r = np.random.default_rng(seed)
    a = np.arange(256) - 128
    p = a[:, None] * a[None, :]
    e = np.rint(r.normal(0, 1, p.shape) * (0.02 * np.abs(p) + 1))
    return np.clip(p + e, -32768, 32767).astype(np.float32).reshape(-1)


def tables(kind, lut, qtype="int8"):
    if kind == "ste":
        return None, None
    if kind == "lre":
        ga, gb = O.lre_tables(lut, qtype)
        return ga, gb
    ga, gb = O.date_tables(lut.reshape(256, 256), 2)
    return ga.reshape(-1), gb.reshape(-1)


GEOMS = [dict(k=3, s=1, p=1, d=1), dict(k=3, s=2, p=1, d=1), dict(k=1, s=1, p=0, d=1),
         dict(k=1, s=2, p=0, d=1), dict(k=7, s=2, p=3, d=1), dict(k=3, s=1, p=2, d=2)]


@pytest.mark.parametrize("kind", ["ste", "lre", "custom"])
@pytest.mark.parametrize("gi", range(len(GEOMS)))
def test_conv2d_int8_forward_backward(kind, gi):
    gm = GEOMS[gi]
    torch.manual_seed(gi)
    lut = perturbed_lut(gi)
    dx, dw = tables(kind, lut)
    layer = at.nn.Conv2d_int8(6, 70, gm["k"], torch.from_numpy(lut).to(DEV), grad=kind,
                              dx=None if dx is None else torch.from_numpy(dx).to(DEV),
                              dw=None if dw is None else torch.from_numpy(dw).to(DEV),
                              bias=True, stride=gm["s"], padding=gm["p"], dilation=gm["d"],
                              weight_bits=6).to(DEV)
    layer.eval()
    x = torch.randn(3, 6, 13, 12, device=DEV)
    with torch.no_grad():
        layer.scale_x.fill_(float(x.abs().max()) / 110.0)     # some activations clip
    xr = x.clone().requires_grad_()
    y = layer(xr)
    k2, s2, p2, d2 = (gm["k"],) * 2, (gm["s"],) * 2, (gm["p"],) * 2, (gm["d"],) * 2
    sx = np.float32(layer.scale_x.item())
    sw = layer.scale_w.cpu().numpy()
    want, ctx = O.conv_int8_forward(x.cpu().numpy(), layer.weight.detach().cpu().numpy(),
                                    layer.bias.detach().cpu().numpy(), lut, sx, sw,
                                    k2, s2, p2, d2, weight_bits=6)
    close(y, want, ctx["yabs"])
    go = torch.randn_like(y)
    y.backward(go)
    tb = None if kind == "ste" else (dx, dw)
    gx, gw, gb = O.conv_int8_backward(go.cpu().numpy(), ctx, sx, sw, kind, tb, k2, s2, p2, d2)
    ax, aw, ab = O.conv_int8_backward(go.cpu().numpy(), ctx, sx, sw, kind, tb, k2, s2, p2, d2,
                                      absolute=True)
    close(xr.grad, gx, ax)
    close(layer.weight.grad, gw, aw)
    close(layer.bias.grad, gb, ab)


@pytest.mark.parametrize("gi", [0, 1, 2])
def test_conv2d_int8_save_image_mode(gi):
    """save_image=True keeps the int8 image instead of the row-offset operand
    and unfolds it again for grad_w: identical forward sums and grad_x, grad_w
    against the oracle (the memory it saves is measured at size by bench.py's
    layer_memory)."""
    gm = GEOMS[gi]
    lut = perturbed_lut(11)
    dx, dw = O.lre_tables(lut)
    outs = []
    for save_image in (False, True):
        torch.manual_seed(3)
        layer = at.nn.Conv2d_int8(16, 32, gm["k"], torch.from_numpy(lut).to(DEV), grad="lre",
                                  dx=torch.from_numpy(dx).to(DEV), dw=torch.from_numpy(dw).to(DEV),
                                  bias=True, stride=gm["s"], padding=gm["p"], dilation=gm["d"],
                                  save_image=save_image).to(DEV).eval()
        x = torch.randn(4, 16, 20, 20, device=DEV, generator=torch.Generator(DEV).manual_seed(1))
        with torch.no_grad():
            layer.scale_x.fill_(float(x.abs().max()) / 120.0)
        xr = x.clone().requires_grad_()
        y = layer(xr)
        go = torch.randn(y.shape, device=DEV, generator=torch.Generator(DEV).manual_seed(2))
        y.backward(go)
        outs.append((y.detach(), xr.grad, layer.weight.grad, layer, x, go))
    (y0, gx0, gw0, l0, x, go), (y1, gx1, gw1, _, _, _) = outs
    assert torch.equal(y0, y1) and torch.equal(gx0, gx1)
    k2, s2, p2, d2 = (gm["k"],) * 2, (gm["s"],) * 2, (gm["p"],) * 2, (gm["d"],) * 2
    sx, sw = np.float32(l0.scale_x.item()), l0.scale_w.cpu().numpy()
    _, ctx = O.conv_int8_forward(x.cpu().numpy(), l0.weight.detach().cpu().numpy(),
                                 l0.bias.detach().cpu().numpy(), lut, sx, sw, k2, s2, p2, d2)
    _, gw, _ = O.conv_int8_backward(go.cpu().numpy(), ctx, sx, sw, "lre", (dx, dw), k2, s2, p2,
                                    d2)
    _, aw, _ = O.conv_int8_backward(go.cpu().numpy(), ctx, sx, sw, "lre", (dx, dw), k2, s2, p2,
                                    d2, absolute=True)
    close(gw1, gw, aw)
    close(gw0, gw, aw)


@pytest.mark.parametrize("kind", ["ste", "lre"])
@pytest.mark.parametrize("gi", [0, 1, 4, 5])
def test_conv2d_int8_depthwise_forward_backward(kind, gi):
    """groups == in == out (MobileNet's depthwise conv) through the depthwise
    LUT kernel, against the oracle's per-channel layer."""
    gm = GEOMS[gi]
    torch.manual_seed(20 + gi)
    lut = perturbed_lut(20 + gi)
    dx, dw = tables(kind, lut)
    C = 12
    layer = at.nn.Conv2d_int8(C, C, gm["k"], torch.from_numpy(lut).to(DEV), grad=kind,
                              dx=None if dx is None else torch.from_numpy(dx).to(DEV),
                              dw=None if dw is None else torch.from_numpy(dw).to(DEV),
                              bias=True, stride=gm["s"], padding=gm["p"], dilation=gm["d"],
                              groups=C).to(DEV)
    layer.eval()
    x = torch.randn(3, C, 13, 12, device=DEV)
    with torch.no_grad():
        layer.scale_x.fill_(float(x.abs().max()) / 110.0)
    xr = x.clone().requires_grad_()
    y = layer(xr)
    k2, s2, p2, d2 = (gm["k"],) * 2, (gm["s"],) * 2, (gm["p"],) * 2, (gm["d"],) * 2
    sx = np.float32(layer.scale_x.item())
    sw = layer.scale_w.cpu().numpy()
    want, ctxs = O.dwconv_int8_forward(x.cpu().numpy(), layer.weight.detach().cpu().numpy(),
                                       layer.bias.detach().cpu().numpy(), lut, sx, sw,
                                       k2, s2, p2, d2)
    close(y, want, O.dwconv_yabs(ctxs))
    go = torch.randn_like(y)
    y.backward(go)
    tb = None if kind == "ste" else (dx, dw)
    gx, gw, gb = O.dwconv_int8_backward(go.cpu().numpy(), ctxs, sx, sw, kind, tb, k2, s2, p2,
                                        d2)
    ax, aw, ab = O.dwconv_int8_backward(go.cpu().numpy(), ctxs, sx, sw, kind, tb, k2, s2, p2,
                                        d2, absolute=True)
    close(xr.grad, gx, ax)
    close(layer.weight.grad, gw, aw)
    close(layer.bias.grad, gb, ab)


@pytest.mark.parametrize("kind", ["ste", "lre", "custom"])
@pytest.mark.parametrize("gi", [0, 1, 2, 5])
def test_conv2d_uint8_forward_backward(kind, gi):
    gm = GEOMS[gi]
    torch.manual_seed(10 + gi)
    v = np.arange(256)
    lut = ((v[:, None] * v[None, :]) & ~63).astype(np.float32).reshape(-1)   # config 5 table
    dx, dw = tables(kind, lut, "uint8")
    wb = 4 if kind == "custom" else 8
    layer = at.nn.Conv2d_uint8(5, 66, gm["k"], torch.from_numpy(lut).to(DEV), grad=kind,
                               dx=None if dx is None else torch.from_numpy(dx).to(DEV),
                               dw=None if dw is None else torch.from_numpy(dw).to(DEV),
                               bias=True, stride=gm["s"], padding=gm["p"], dilation=gm["d"],
                               weight_bits=wb).to(DEV)
    x = torch.randn(2, 5, 11, 13, device=DEV) + 0.4
    layer.train()
    with torch.no_grad():
        layer(x)                                      # one EMA step sets non-trivial qparams
    layer.eval()
    xr = x.clone().requires_grad_()
    y = layer(xr)
    k2, s2, p2, d2 = (gm["k"],) * 2, (gm["s"],) * 2, (gm["p"],) * 2, (gm["d"],) * 2
    want, ctx = O.conv_uint8_forward(
        x.cpu().numpy(), layer.weight.detach().cpu().numpy(), layer.bias.detach().cpu().numpy(),
        lut, np.float32(layer.scale_x.item()), np.float32(layer.zero_x.item()),
        layer.scale_w.cpu().numpy(), layer.zero_w.cpu().numpy(), k2, s2, p2, d2,
        qmax_w=2 ** wb - 1)
    close(y, want, ctx["yabs"])
    go = torch.randn_like(y)
    y.backward(go)
    tb = None if kind == "ste" else (dx, dw)
    args = (go.cpu().numpy(), ctx, np.float32(layer.scale_x.item()), layer.scale_w.cpu().numpy(),
            kind, tb, k2, s2, p2, d2)
    gx, gw, gb = O.conv_uint8_backward(*args)
    ax, aw, ab = O.conv_uint8_backward(*args, absolute=True)
    close(xr.grad, gx, ax)
    close(layer.weight.grad, gw, aw)
    close(layer.bias.grad, gb, ab)


@pytest.mark.parametrize("kind", ["ste", "lre", "custom"])
@pytest.mark.parametrize("shape", [(1, 1, 0, 7, 9), (3, 2, 1, 12, 12)])
def test_conv2d_uint8_fused_matches_composition(kind, shape):
    """The fused layer path (one Function: uint8 image, in-place zero-point
    correction and dequant, fused backward terms) against the reference's
    composition of the public pieces (static_quantize_uint8, the conv-level
    Function, tap_sum and the correction as torch ops, nn/Conv2d_uint8.py:
    257-325): forward and every gradient, without bias, for a 1x1 conv with
    L % 4 != 0 and a strided 3x3 conv."""
    from approxtorch_amd.nn import bgemm_uint8, quantization
    k, s, p, H, W = shape
    torch.manual_seed(21)
    v = np.arange(256)
    lut = torch.from_numpy(((v[:, None] * v[None, :]) & ~63).astype(np.float32).reshape(-1)).to(DEV)
    dx, dw = tables(kind, lut.cpu().numpy(), "uint8")
    tx = None if dx is None else torch.from_numpy(dx).to(DEV)
    tw = None if dw is None else torch.from_numpy(dw).to(DEV)
    layer = at.nn.Conv2d_uint8(6, 20, k, lut, grad=kind, dx=tx, dw=tw, bias=False, stride=s,
                               padding=p, weight_bits=4 if kind == "custom" else 8).to(DEV)
    x = torch.randn(2, 6, H, W, device=DEV) + 0.3
    layer.train()
    with torch.no_grad():
        layer(x)
    layer.eval()
    x1 = x.clone().requires_grad_()
    y1 = layer(x1)
    go = torch.randn_like(y1)
    y1.backward(go)
    g1x, g1w = x1.grad.clone(), layer.weight.grad.clone()
    layer.weight.grad = None

    x2 = x.clone().requires_grad_()
    geom = ((k, k), layer.stride, layer.padding, layer.dilation, 1)
    xq = quantization.static_quantize_uint8(x2, layer.scale_x, layer.zero_x, 0, 255)
    wq = quantization.static_quantize_uint8(layer.weight, layer.scale_w, layer.zero_w, 0,
                                            layer.qmax_w, ch_axis=0)
    wu = wq.view(20, -1)
    if kind == "ste":
        y = bgemm_uint8.conv2d_uint8_ste(xq, wu, lut, layer.zero_x, geom)
    elif kind == "lre":
        y = bgemm_uint8.conv2d_uint8_lre(xq, wu, lut, tx, tw, layer.zero_x, geom)
    else:
        y = bgemm_uint8.conv2d_uint8_custom(xq, wu, lut, tx, tw, layer.zero_x, geom)
    xsum = bgemm_uint8.tap_sum(xq, layer.zero_x, geom)
    zw = layer.zero_w.view(1, -1, 1)
    y = y - zw * xsum.unsqueeze(1) - (layer.zero_x * wu.sum(dim=1)).view(1, -1, 1) \
        + wu.shape[1] * layer.zero_x * zw
    y2 = y.view_as(y1) * (layer.scale_x * layer.scale_w).view(1, -1, 1, 1)
    y2.backward(go)
    # identical fp32 operations in the same order: the forward is bitwise equal
    assert torch.equal(y1, y2)
    for a, b in ((g1x, x2.grad), (g1w, layer.weight.grad)):
        tol = 1e-5 * b.abs().max().item() + 1e-4
        assert (a - b).abs().max().item() <= tol


def test_train_mode_ema_matches_reference_rules():
    torch.manual_seed(3)
    lut = torch.from_numpy(perturbed_lut(3)).to(DEV)
    layer = at.nn.Conv2d_int8(4, 8, 3, lut, padding=1, scale_momentum=0.1, weight_bits=5).to(DEV)
    layer.train()
    sx = np.float32(layer.scale_x.item())
    sw = layer.scale_w.cpu().numpy()
    with torch.no_grad():
        layer.weight[2].zero_()
    for step in range(3):
        x = torch.randn(2, 4, 9, 9, device=DEV) * (step + 1)
        w = layer.weight.detach().cpu().numpy()
        layer(x)
        sx = O.ema_absmax(x.cpu().numpy(), sx, 0.1)
        sw = O.weight_scale_ema(w, sw, 0.1, 15)
        assert layer.scale_x.item() == sx
        assert np.array_equal(layer.scale_w.cpu().numpy(), sw)
    layer.freeze_scale()
    before = layer.scale_x.item()
    layer(torch.randn(2, 4, 9, 9, device=DEV) * 50)
    assert layer.scale_x.item() == before


def test_convert_model_training_step_runs_and_learns():
    torch.manual_seed(0)
    net = torch.nn.Sequential(
        torch.nn.Conv2d(3, 16, 3, padding=1), torch.nn.ReLU(),
        torch.nn.Conv2d(16, 32, 3, padding=1, stride=2), torch.nn.ReLU(),
        torch.nn.Conv2d(32, 32, 3, padding=1), torch.nn.ReLU(),
        torch.nn.AdaptiveAvgPool2d(1), torch.nn.Flatten(), torch.nn.Linear(32, 10)).to(DEV)
    a = np.arange(256) - 128
    lut = torch.tensor(((a[:, None] * a[None, :]) >> 4 << 4).reshape(-1),
                       dtype=torch.float32, device=DEV)
    net = at.convert_model(net, lut, qtype="int8", grad="ste", scale_momentum=0.1)
    assert isinstance(net[0], torch.nn.Conv2d) and isinstance(net[2], at.nn.Conv2d_int8)
    opt = torch.optim.SGD(net.parameters(), lr=0.05, momentum=0.9)
    x = torch.randn(16, 3, 16, 16, device=DEV)
    y = torch.randint(0, 10, (16,), device=DEV)
    losses = []
    for _ in range(15):
        opt.zero_grad()
        loss = torch.nn.functional.cross_entropy(net(x), y)
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert np.isfinite(losses).all()
    assert losses[-1] < losses[0]
