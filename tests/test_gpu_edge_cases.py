"""The reference's own edge-case checks for the conv path, restated against
the CPU oracle (csrc/claude/verify_correctness.py:200-300,
csrc/claude/test_conv_decoupled.py:199-222):

  D  adversarial padding: dw[128] = 1e4 on a padding-dominated 5x5 image
  E  the seed-7 fuzz over 30 random geometries (groups 1 / depthwise, STE / LRE)
  F  int16-boundary and fp32-fallback LUTs; channels_last and storage-offset inputs
  the 13-geometry LRE sweep and 9 STE geometries (batch 1, H != W, no bias, ...)

Forward values and gradients are compared with the oracle within rel 1e-5 of
the sum of |terms| / abs 1e-4; LUT sums are exact."""
import random
import zlib

import numpy as np
import pytest
import torch

import approxtorch_amd as at
from approxtorch_amd.backend import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-5, 1e-4


def close(got, want, absref, what=""):
    got = got.detach().double().cpu().numpy() if torch.is_tensor(got) else np.asarray(got)
    excess = np.abs(got - want) - (ATOL + RTOL * np.asarray(absref))
    assert excess.max() <= 0, f"{what} max excess {excess.max():.3g}"


ii = np.arange(256, dtype=np.float32) - 128
EXACT_LUT = (ii[:, None] * ii[None, :]).reshape(-1)


def module(C, O_, k, s, p, d, g, mode, lut, dx=None, dw=None, bias=True):
    """make_module of verify_correctness.py:56-67: train mode, frozen scale_x = 0.02."""
    kw = {}
    if mode == "lre":
        kw = dict(dx=torch.as_tensor(dx, device=DEV), dw=torch.as_tensor(dw, device=DEV))
    m = at.nn.Conv2d_int8(C, O_, k, torch.as_tensor(lut, device=DEV), grad=mode, bias=bias,
                          stride=s, padding=p, dilation=d, groups=g, **kw).to(DEV)
    m.train()
    m.update_scale = False
    with torch.no_grad():
        m.scale_x.fill_(0.02)
    return m


def check_module(m, x, go, lut, tables, what):
    """Forward + backward of a Conv2d_int8 against the oracle's layer."""
    xr = x.detach().clone().requires_grad_()
    y = m(xr)
    y.backward(go)
    k, s, p, d = m.kernel_size, m.stride, m.padding, m.dilation
    sx = np.float32(m.scale_x.item())
    sw = m.scale_w.cpu().numpy()
    b = None if m.bias is None else m.bias.detach().cpu().numpy()
    w = m.weight.detach().cpu().numpy()
    gon = go.cpu().numpy()
    if m.groups == 1:
        want, ctx = O.conv_int8_forward(x.cpu().numpy(), w, b, lut, sx, sw, k, s, p, d,
                                        m.weight_bits)
        yabs = ctx["yabs"]
        back = lambda a: O.conv_int8_backward(gon, ctx, sx, sw, m.grad, tables, k, s, p, d,
                                              absolute=a)
    else:
        want, ctx = O.dwconv_int8_forward(x.cpu().numpy(), w, b, lut, sx, sw, k, s, p, d,
                                          m.weight_bits)
        yabs = O.dwconv_yabs(ctx)
        back = lambda a: O.dwconv_int8_backward(gon, ctx, sx, sw, m.grad, tables, k, s, p, d,
                                                absolute=a)
    close(y, want, yabs, f"{what} y")
    (gx, gw, gb), (ax, aw, ab) = back(False), back(True)
    close(xr.grad, gx, ax, f"{what} grad_x")
    close(m.weight.grad, gw, aw, f"{what} grad_w")
    if m.bias is not None:
        close(m.bias.grad, gb, ab, f"{what} grad_b")


# ------------------------------------------------------------------ D
@pytest.mark.parametrize("C,O_,g", [(8, 12, 1), (12, 12, 12)])
def test_adversarial_padding_dw128(C, O_, g):
    """verify_correctness.py:200-223: with dw[128] = 1e4 every padded tap
    dominates grad_w; any slip in the padding index blows past the bound."""
    r = np.random.default_rng(200 + g)
    lut = r.integers(-127 * 127, 127 * 127, 65536).astype(np.float32)
    dx = r.standard_normal(256).astype(np.float32)
    dw = r.standard_normal(256).astype(np.float32)
    dw[128] = 1e4
    B, H, W = 2, 5, 5
    xv = r.integers(-127, 128, (B, C, H, W)).astype(np.float32)
    wv = r.integers(-127, 128, (O_, (C // g) * 9)).astype(np.float32)
    x, w = torch.as_tensor(xv, device=DEV).requires_grad_(), \
        torch.as_tensor(wv, device=DEV).requires_grad_()
    y = at.nn.bgemm_int8.conv2d_int8_lre(x, w, torch.as_tensor(lut, device=DEV),
                                         torch.as_tensor(dx, device=DEV),
                                         torch.as_tensor(dw, device=DEV),
                                         ((3, 3), (1, 1), (2, 2), (1, 1), g))
    go = r.standard_normal((B, O_, 49)).astype(np.float32)
    y.backward(torch.as_tensor(go, device=DEV).view_as(y))
    k, s, p, d = (3, 3), (1, 1), (2, 2), (1, 1)
    if g == 1:
        xi = O.im2col_index(O.image_index(xv.astype(np.int8)), k, s, p, d, 128)
        wi = (wv + 128).astype(np.uint8)
        _, gw = O.gemm_grads(go, xi, wi, "lre", (dx, dw))
        _, aw = O.gemm_grads(go, xi, wi, "lre", (dx, dw), absolute=True)
    else:
        gw, aw = np.zeros((C, 9)), np.zeros((C, 9))
        for c in range(C):
            xi = O.im2col_index(O.image_index(xv[:, c:c + 1].astype(np.int8)), k, s, p, d, 128)
            wi = (wv[c:c + 1] + 128).astype(np.uint8)
            gw[c] = O.gemm_grads(go[:, c:c + 1], xi, wi, "lre", (dx, dw))[1][0]
            aw[c] = O.gemm_grads(go[:, c:c + 1], xi, wi, "lre", (dx, dw), absolute=True)[1][0]
    close(w.grad, gw, aw, "grad_w")
    # the padded taps carry most of the gradient: the check is not vacuous
    assert np.abs(gw).max() > 1e3


# ------------------------------------------------------------------ E
def _fuzz_configs():
    """The draw sequence of verify_correctness.py:226-253 (random.seed(7))."""
    rnd = random.Random(7)
    out = []
    for _ in range(30):
        g1 = rnd.random() < 0.5
        k = rnd.choice([1, 2, 3, 4, 5])
        s = rnd.choice([1, 2, 3])
        p = rnd.choice([0, 1, 2])
        d = rnd.choice([1, 2]) if k > 1 else 1
        C = rnd.randint(1, 48)
        O_ = rnd.randint(1, 48) if g1 else C
        g = 1 if g1 else C
        mode = rnd.choice(["ste", "lre"])
        bias = rnd.random() < 0.7
        keff = d * (k - 1) + 1
        H = rnd.randint(keff, 23)
        W = rnd.randint(keff, 23)
        if (H + 2 * p - keff) < 0 or (W + 2 * p - keff) < 0:
            continue
        B = rnd.randint(1, 4)
        out.append((B, C, O_, H, W, k, s, p, d, g, mode, bias))
    return out


FUZZ = _fuzz_configs()


@pytest.mark.parametrize("cfg", FUZZ, ids=[f"fuzz{i}" for i in range(len(FUZZ))])
def test_fuzz_seed7(cfg):
    B, C, O_, H, W, k, s, p, d, g, mode, bias = cfg
    r = np.random.default_rng(zlib.crc32(repr(cfg).encode()))
    dx = r.standard_normal(256).astype(np.float32) if mode == "lre" else None
    dw = r.standard_normal(256).astype(np.float32) if mode == "lre" else None
    m = module(C, O_, k, s, p, d, g, mode, EXACT_LUT, dx, dw, bias)
    x = torch.as_tensor(r.standard_normal((B, C, H, W)).astype(np.float32), device=DEV)
    with torch.no_grad():
        shape = m(x).shape
    go = torch.as_tensor(r.standard_normal(shape).astype(np.float32), device=DEV)
    check_module(m, x, go, EXACT_LUT, None if mode == "ste" else (dx, dw), str(cfg))


# ------------------------------------------------------------------ F
def test_int16_boundary_and_fp32_fallback_luts():
    """verify_correctness.py:272-290 on the depthwise op: an int16-boundary LUT
    (+-32767) takes the integer path, one entry of 32768 forces the fp32
    fallback; both equal the sequential fp32 sum over taps bitwise."""
    r = np.random.default_rng(272)
    x8 = r.integers(-127, 128, (2, 8, 12, 12)).astype(np.int8)
    w = r.integers(-127, 128, (8, 9)).astype(np.float32)
    edge = np.full((256, 256), 32767.0, np.float32)
    edge[::2] = -32767.0
    bad = edge.copy()
    bad[0, 0] = 32768.0
    xi = O.im2col_index(O.image_index(x8), (3, 3), (1, 1), (1, 1), (1, 1), 128)
    xi = xi.reshape(2, 8, 9, -1)
    wi = (w + 128).astype(np.int64)
    for lut in (edge, bad):
        y, _ = ops.dwconv_fake_int8_claude(torch.as_tensor(x8, device=DEV),
                                           torch.as_tensor(w, device=DEV),
                                           torch.as_tensor(lut, device=DEV), 3, 1, 1, 1)
        lf = lut.reshape(-1)
        acc = np.zeros((2, 8, xi.shape[-1]), np.float32)
        for tp in range(9):
            acc = (acc + lf[xi[:, :, tp].astype(np.int64) * 256 + wi[None, :, tp, None]]
                   ).astype(np.float32)
        assert np.array_equal(y.flatten(2).cpu().numpy(), acc)


@pytest.mark.parametrize("g,C", [(1, 16), (16, 16)])
def test_non_contiguous_inputs(g, C):
    """verify_correctness.py:292-300: channels_last and storage-offset inputs
    give the same output as the contiguous input."""
    r = np.random.default_rng(292 + g)
    lut = r.integers(-127 * 127, 127 * 127, 65536).astype(np.float32)
    m = module(C, 16, 3, 1, 1, 1, g, "lre", lut, r.standard_normal(256).astype(np.float32),
               r.standard_normal(256).astype(np.float32))
    xb = torch.as_tensor(r.standard_normal((4, C, 14, 14)).astype(np.float32), device=DEV)
    y_c = m(xb)
    y_cl = m(xb.to(memory_format=torch.channels_last))
    y_sl = m(torch.cat([xb, xb], 0)[4:])
    assert torch.equal(y_c, y_cl) and torch.equal(y_c, y_sl)


# ------------------------------------------------- test_conv_decoupled sweep
SWEEP = [  # (tag, B, C, H, W, O, k, s, p, d, bias, mode)
    ("k3 s1 p1 resnet block", 8, 64, 28, 28, 64, 3, 1, 1, 1, True, "lre"),
    ("k3 s2 p1 downsample", 8, 64, 28, 28, 128, 3, 2, 1, 1, True, "lre"),
    ("k1 s1 p0 bottleneck", 8, 64, 28, 28, 256, 1, 1, 0, 1, True, "lre"),
    ("k1 s2 p0 shortcut", 8, 64, 28, 28, 128, 1, 2, 0, 1, True, "lre"),
    ("k7 s2 p3 stem C=3", 4, 3, 64, 64, 32, 7, 2, 3, 1, True, "lre"),
    ("k5 s1 p2", 4, 16, 20, 20, 24, 5, 1, 2, 1, True, "lre"),
    ("k3 s1 p2 d2 dilated", 4, 16, 20, 20, 24, 3, 1, 2, 2, True, "lre"),
    ("k3 s1 p0 no-pad", 4, 16, 20, 20, 24, 3, 1, 0, 1, True, "lre"),
    ("k3 s1 p1 no bias", 4, 16, 20, 20, 24, 3, 1, 1, 1, False, "lre"),
    ("k3 s1 p1 batch1", 1, 16, 20, 20, 24, 3, 1, 1, 1, True, "lre"),
    ("k1 s1 p0 batch1", 1, 16, 20, 20, 24, 1, 1, 0, 1, True, "lre"),
    ("k3 s1 p1 H!=W", 4, 16, 24, 18, 24, 3, 1, 1, 1, True, "lre"),
    ("k3 s1 p1 cifar tiny", 16, 16, 32, 32, 16, 3, 1, 1, 1, True, "lre"),
    ("ste k3 s1 p1 resnet block", 8, 64, 28, 28, 64, 3, 1, 1, 1, True, "ste"),
    ("ste k3 s2 p1 downsample", 8, 64, 28, 28, 128, 3, 2, 1, 1, True, "ste"),
    ("ste k1 s1 p0 bottleneck", 8, 64, 28, 28, 256, 1, 1, 0, 1, True, "ste"),
    ("ste k1 s2 p0 shortcut", 8, 64, 28, 28, 128, 1, 2, 0, 1, True, "ste"),
    ("ste k7 s2 p3 stem C=3", 4, 3, 64, 64, 32, 7, 2, 3, 1, True, "ste"),
    ("ste k3 s1 p2 d2 dilated", 4, 16, 20, 20, 24, 3, 1, 2, 2, True, "ste"),
    ("ste k3 s1 p1 no bias", 4, 16, 20, 20, 24, 3, 1, 1, 1, False, "ste"),
    ("ste k3 s1 p1 batch1", 1, 16, 20, 20, 24, 3, 1, 1, 1, True, "ste"),
    ("ste k3 s1 p1 H!=W", 4, 16, 24, 18, 24, 3, 1, 1, 1, True, "ste"),
]


@pytest.mark.parametrize("case", SWEEP, ids=[c[0].replace(" ", "_") for c in SWEEP])
def test_decoupled_geometry_sweep(case):
    """test_conv_decoupled.py:113-222: random LUT in +-127^2, random slope
    tables, scale_x = 0.02, inputs ~ 2 N(0,1) (some clip)."""
    tag, B, C, H, W, O_, k, s, p, d, bias, mode = case
    r = np.random.default_rng(zlib.crc32(tag.encode()))
    lut = r.integers(-127 * 127, 127 * 127, 65536).astype(np.float32)
    dx = r.standard_normal(256).astype(np.float32) if mode == "lre" else None
    dw = r.standard_normal(256).astype(np.float32) if mode == "lre" else None
    m = module(C, O_, k, s, p, d, 1, mode, lut, dx, dw, bias)
    x = torch.as_tensor(r.standard_normal((B, C, H, W)).astype(np.float32) * 2.0, device=DEV)
    with torch.no_grad():
        shape = m(x).shape
    go = torch.as_tensor(r.standard_normal(shape).astype(np.float32), device=DEV)
    check_module(m, x, go, lut, None if mode == "ste" else (dx, dw), tag)
