"""GPU tests of the public API surface: the reference's autograd Functions at
GEMM and conv level (nn/bgemm_int8.py, nn/bgemm_uint8.py), every op schema
registered under torch.ops.approxtorch, the argument checks the reference's
TORCH_CHECKs make, and the autograd hazards around in-place statistic
updates and cached LUT images.  Results are compared with the CPU oracle:
integer sums bit-exact, gradients within rel 1e-5 (against the sum of
|terms|, the bound any fp32 summation order meets) / abs 1e-4."""
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


def gen(key):
    return np.random.default_rng(zlib.crc32(repr(key).encode()))


def t(a, dtype=None, grad=False):
    x = torch.as_tensor(np.ascontiguousarray(a), device=DEV, dtype=dtype)
    return x.requires_grad_() if grad else x


def close(got, want, absref):
    got = got.detach().double().cpu().numpy() if torch.is_tensor(got) else np.asarray(got)
    excess = np.abs(got - want) - (ATOL + RTOL * absref)
    assert excess.max() <= 0, f"max excess {excess.max():.3g}"


def asym_lut():
    v = np.arange(256)
    return (37 * v[:, None] - 19 * v[None, :] + 11).reshape(-1).astype(np.float32)


def perturbed_lut(seed):
    r = np.random.default_rng(seed)
    a = np.arange(256) - 128
    p = a[:, None] * a[None, :]
    e = np.rint(r.normal(0, 1, p.shape) * (0.02 * np.abs(p) + 1))
    return np.clip(p + e, -32768, 32767).astype(np.float32).reshape(-1)


def pair_tables():
    # 2-D custom tables (test_conv_custom_grad.py:41-44 recipe)
    rr, cc = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
    dxl = (rr * 1009 + cc * 7 + (rr * cc) % 31).astype(np.float32) / 1000.0
    return dxl, dxl.T.copy()


def slope_tables():
    # nonlinear LRE slopes (test_bgemm_lre_naive.py:55-57 recipe)
    q = np.arange(256, dtype=np.float32) - 128
    return ((0.0003 * q * q - 0.07 * q + 1.25).astype(np.float32),
            (2.5 * np.sin(0.031 * q) + 0.004 * q).astype(np.float32))


def grads_ref(go, xi, wi, kind, tables, signed):
    g, gw = O.gemm_grads(go, xi, wi, kind, tables, signed)
    if kind == "custom":
        ab = (np.abs(tables[0]), np.abs(tables[1]))
    elif kind == "lre":
        ab = (np.abs(tables[0]), np.abs(tables[1]))
    else:
        ab = None
    ag, agw = O.gemm_grads(np.abs(go), xi, wi, kind if kind != "ste" else "lre",
                           ab if ab is not None else
                           (np.abs(np.arange(256) - (128 if signed else 0)).astype(np.float32),) * 2,
                           signed)
    return g, gw, ag, agw


# --------------------------------------------------- GEMM-level Functions
@pytest.mark.parametrize("kind", ["ste", "lre", "custom"])
@pytest.mark.parametrize("qtype", ["int8", "uint8"])
def test_bgemm_functions_forward_backward(kind, qtype):
    """bgemm_{int8,uint8}_{ste,lre,custom} (nn/bgemm_int8.py:5-84,
    nn/bgemm_uint8.py:27-114) on integer-valued fp32 operands."""
    r = gen(("bgemm_fn", kind, qtype))
    N, K, L, Oc = 2, 37, 53, 19
    off = 128 if qtype == "int8" else 0
    lo, hi = (-127, 128) if qtype == "int8" else (0, 256)
    xv = r.integers(lo, hi, (N, K, L)).astype(np.float32)
    wv = r.integers(lo, hi, (Oc, K)).astype(np.float32)
    xi, wi = (xv + off).astype(np.uint8), (wv + off).astype(np.uint8)
    lut = asym_lut() if qtype == "int8" else ((np.arange(256)[:, None] * np.arange(256)[None, :])
                                              & ~63).reshape(-1).astype(np.float32)
    mod = at.nn.bgemm_int8 if qtype == "int8" else at.nn.bgemm_uint8
    x, w, lt = t(xv, grad=True), t(wv, grad=True), t(lut)
    if kind == "ste":
        tables = None
        y = getattr(mod, f"bgemm_{qtype}_ste")(x, w, lt)
    elif kind == "lre":
        tables = slope_tables()
        y = getattr(mod, f"bgemm_{qtype}_lre")(x, w, lt, t(tables[0]), t(tables[1]))
    else:
        tables = pair_tables()
        y = getattr(mod, f"bgemm_{qtype}_custom")(x, w, lt, t(tables[0].reshape(-1)),
                                                  t(tables[1].reshape(-1)))
    assert np.array_equal(y.detach().cpu().numpy().astype(np.int64), O.lut_gemm_i64(xi, wi, lut))
    go = r.standard_normal(y.shape).astype(np.float32)
    y.backward(t(go))
    gx, gw, ax, aw = grads_ref(go, xi, wi, kind, tables, qtype == "int8")
    close(x.grad, gx, ax)
    close(w.grad, gw, aw)


def test_bgemm_uint8_is_forward_only():
    x = t(np.ones((1, 3, 4), np.float32), grad=True)
    w = t(np.ones((2, 3), np.float32), grad=True)
    y = at.nn.bgemm_uint8.bgemm_uint8(x, w, t(asym_lut()))
    assert torch.equal(y, torch.full_like(y, float(3 * asym_lut()[257])))
    with pytest.raises(NotImplementedError, match="forward-only"):
        y.sum().backward()


# --------------------------------------------------- conv-level Functions
CONV_GEOMS = [((3, 3), (1, 1), (1, 1), (1, 1)), ((3, 3), (2, 2), (1, 1), (1, 1)),
              ((1, 1), (1, 1), (0, 0), (1, 1)), ((3, 3), (1, 1), (2, 2), (2, 2)),
              ((5, 3), (2, 1), (2, 1), (1, 1))]


@pytest.mark.parametrize("kind", ["ste", "lre", "custom"])
@pytest.mark.parametrize("gi", range(len(CONV_GEOMS)))
def test_conv2d_int8_functions(kind, gi):
    """conv2d_int8_{ste,lre,custom} (nn/bgemm_int8.py:87-298) on a quantized
    image: forward bit-exact, padded taps index 128; backward = fold of the
    unfolded estimator gradient."""
    k, s, p, d = CONV_GEOMS[gi]
    r = gen(("conv_fn", kind, gi))
    N, C, H, W, Oc = 2, 5, 11, 9, 23
    xv = r.integers(-127, 128, (N, C, H, W)).astype(np.float32)
    K = C * k[0] * k[1]
    wv = r.integers(-127, 128, (Oc, K)).astype(np.float32)
    lut = perturbed_lut(gi)
    x, w = t(xv, grad=True), t(wv, grad=True)
    geom = (k, s, p, d, 1)
    if kind == "ste":
        tables = None
        y = at.nn.bgemm_int8.conv2d_int8_ste(x, w, t(lut), geom)
    elif kind == "lre":
        tables = slope_tables()
        y = at.nn.bgemm_int8.conv2d_int8_lre(x, w, t(lut), t(tables[0]), t(tables[1]), geom)
    else:
        tables = pair_tables()
        y = at.nn.bgemm_int8.conv2d_int8_custom(x, w, t(lut), t(tables[0].reshape(-1)),
                                                t(tables[1].reshape(-1)), geom)
    xi = O.im2col_index(O.image_index(xv.astype(np.int8)), k, s, p, d, 128)
    wi = (wv + 128).astype(np.uint8)
    want = O.lut_gemm_i64(xi, wi, lut)
    assert np.array_equal(y.detach().cpu().numpy().reshape(want.shape).astype(np.int64), want)
    go = r.standard_normal(y.shape).astype(np.float32)
    y.backward(t(go))
    gcol, gw, acol, aw = grads_ref(go.reshape(N, Oc, -1), xi, wi, kind, tables, True)
    close(x.grad, O.fold(gcol, (N, C, H, W), k, s, p, d), O.fold(acol, (N, C, H, W), k, s, p, d))
    close(w.grad, gw, aw)


# ------------------------------------------------ registered op schemas
def test_every_reference_schema_is_registered():
    names = ["bgemm_fake_int8_forward_cuda_claude", "bgemm_fake_int8_forward_cuda_claude_cfg",
             "bgemm_fake_int8_forward_cuda_claude_save", "bgemm_fake_uint8_forward_cuda_claude",
             "bgemm_fake_uint8_forward_cuda_claude_cfg", "bgemm_fake_uint8_forward_cuda_claude_save",
             "gemm_fake_int8_forward_cuda_claude", "gemm_fake_int8_forward_cuda_claude_cfg",
             "gemm_fake_int8_forward_cuda_claude_save", "gemm_fake_uint8_forward_cuda_claude",
             "gemm_fake_uint8_forward_cuda_claude_cfg", "gemm_fake_uint8_forward_cuda_claude_save",
             "dwconv_fake_int8_claude", "im2col_u8", "lut_map", "lut_map_pad",
             "bgemm_lre_backward_claude", "bgemm_lre_backward_claude_cfg",
             "bgemm_lre_backward_claude_im2col", "bgemm_custom_grad_uint8_dx",
             "bgemm_custom_grad_uint8_dw", "bgemm_custom_grad_int8_dx", "bgemm_custom_grad_int8_dw",
             "fakequant_per_tensor_claude", "fakequant_per_tensor_backward_claude",
             "fakequant_per_tensor_asymmetric_claude",
             "fakequant_per_tensor_asymmetric_backward_claude"]
    for n in names:
        assert hasattr(getattr(torch.ops.approxtorch, n), "default"), n


@pytest.mark.parametrize("qtype", ["int8", "uint8"])
@pytest.mark.parametrize("variant", ["", "_cfg", "_save"])
def test_gemm_fake_schemas(qtype, variant):
    """torch.ops.approxtorch.gemm_fake_{int8,uint8}_forward_cuda_claude{,_cfg,_save}
    (csrc/claude/gemm.cu:292-307): y[m,n] = sum_k lut[idx(A[m,k])][idx(B[k,n])]."""
    r = gen(("gemm2d", qtype, variant))
    M, K, Nn = 70, 45, 33
    off = 128 if qtype == "int8" else 0
    lo, hi = (-128, 128) if qtype == "int8" else (0, 256)
    A = r.integers(lo, hi, (M, K)).astype(np.float32)
    B = r.integers(lo, hi, (K, Nn)).astype(np.float32)
    lut = asym_lut()
    op = getattr(torch.ops.approxtorch, f"gemm_fake_{qtype}_forward_cuda_claude{variant}").default
    args = (t(A), t(B), t(lut)) + ((3,) if variant == "_cfg" else ())
    out = op(*args)
    y = out[0] if variant == "_save" else out
    ai, bi = (A + off).astype(np.uint8), (B + off).astype(np.uint8)
    want = O.lut_gemm_i64(ai[:, :, None], bi.T, lut)[:, :, 0]
    assert np.array_equal(y.cpu().numpy().astype(np.int64), want)
    if variant == "_save":
        assert np.array_equal(out[1].cpu().numpy(), ai)
        assert np.array_equal(out[2].cpu().numpy(), bi.T)


def test_dwconv_schema():
    """torch.ops.approxtorch.dwconv_fake_int8_claude (csrc/claude/dwconv_claude.cu:279-285)
    equals the LUT-BGEMM run per channel with padded taps at index 128."""
    r = gen("dw_schema")
    N, C, H, W = 2, 6, 10, 7
    k, s, p, d = (3, 3), (2, 1), (1, 1), (1, 1)
    xv = r.integers(-128, 128, (N, C, H, W)).astype(np.int8)
    wv = r.integers(-127, 128, (C, 9)).astype(np.float32)
    lut = perturbed_lut(5)
    y, wq = torch.ops.approxtorch.dwconv_fake_int8_claude.default(
        t(xv), t(wv), t(lut), *k, *s, *p, *d)
    for c in range(C):
        xi = O.im2col_index(O.image_index(xv[:, c:c + 1]), k, s, p, d, 128)
        want = O.lut_gemm_i64(xi, (wv[c:c + 1] + 128).astype(np.uint8), lut)
        assert np.array_equal(y[:, c].reshape(N, -1).cpu().numpy().astype(np.int64), want[:, 0])
    assert np.array_equal(wq.cpu().numpy(), (wv + 128).astype(np.uint8))


@pytest.mark.parametrize("xdtype", ["int8", "uint8", "float32"])
def test_lre_backward_cfg_and_im2col_schemas(xdtype):
    """bgemm_lre_backward_claude_cfg / _im2col (csrc/claude/bgemm_lre_backward_claude.cu:
    892-908): the im2col variant takes the pre-unfold image and maps padded taps
    to dw[128]; both return (grad_x [N,K,L] unfolded, grad_w [K,O])."""
    r = gen(("lre_schema", xdtype))
    N, C, H, W, Oc = 2, 4, 9, 8, 21
    k, s, p, d = (3, 3), (1, 2), (1, 1), (1, 1)
    K = C * 9
    xi_img = r.integers(0, 256, (N, C, H, W), dtype=np.uint8)
    wi = r.integers(0, 256, (Oc, K), dtype=np.uint8)
    if xdtype == "uint8":
        ximg = xi_img
    elif xdtype == "int8":
        ximg = (xi_img.astype(np.int16) - 128).astype(np.int8)
    else:
        ximg = xi_img.astype(np.float32) - 128
    dx, dw = slope_tables()
    xcol = O.im2col_index(xi_img, k, s, p, d, 128)
    Lc = xcol.shape[2]
    go = r.standard_normal((N, Oc, Lc)).astype(np.float32)
    wT = np.ascontiguousarray(wi.T)
    gx, gw = torch.ops.approxtorch.bgemm_lre_backward_claude_im2col.default(
        t(go), t(ximg), t(wT), t(dx), t(dw), *k, *s, *p, *d)
    ex, ew = O.gemm_grads(go, xcol, wi, "lre", (dx, dw))
    ax, aw = O.gemm_grads(np.abs(go), xcol, wi, "lre", (np.abs(dx), np.abs(dw)))
    close(gx, ex, ax)
    close(gw, ew.T, aw.T)
    gx2, gw2 = torch.ops.approxtorch.bgemm_lre_backward_claude_cfg.default(
        t(go), t(xcol), t(wT), t(dx), t(dw), 2)
    close(gx2, ex, ax)
    close(gw2, ew.T, aw.T)


def test_lre_backward_degenerate_shapes_return_zeros():
    go = torch.zeros(0, 4, 5, device=DEV)
    x = torch.zeros(0, 3, 5, dtype=torch.uint8, device=DEV)
    w = torch.zeros(3, 4, dtype=torch.uint8, device=DEV)
    tb = torch.ones(256, device=DEV)
    gx, gw = ops.bgemm_lre_backward_claude(go, x, w, tb, tb)
    assert gx.shape == (0, 3, 5) and gw.shape == (3, 4) and not gw.any()


# -------------------------------------------------------- argument checks
def test_fakequant_rejects_inputs_the_reference_rejects():
    """csrc/claude/quantization.cu:190-193,226-232: RuntimeError, no launch."""
    x = torch.randn(64, device=DEV)
    s = torch.tensor(0.1, device=DEV)
    with pytest.raises(RuntimeError, match="float32"):
        ops.fakequant_per_tensor(x.double(), s, -127, 127)
    with pytest.raises(RuntimeError, match="CUDA"):
        ops.fakequant_per_tensor(x, s.cpu(), -127, 127)
    with pytest.raises(RuntimeError, match="scalar"):
        ops.fakequant_per_tensor(x, torch.ones(2, device=DEV), -127, 127)
    with pytest.raises(RuntimeError, match="float32"):
        ops.fakequant_per_tensor(x, s.double(), -127, 127)
    q, m, _ = ops.fakequant_per_tensor(x, s, -127, 127)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        ops.fakequant_per_tensor_backward(x[:32], m, s)
    with pytest.raises(RuntimeError, match="bool"):
        ops.fakequant_per_tensor_backward(x, m.to(torch.uint8), s)
    with pytest.raises(RuntimeError, match="CUDA"):
        ops.fakequant_per_tensor_backward(x, m, s.cpu())
    with pytest.raises(RuntimeError, match="float32"):
        ops.fakequant_rows(x.view(1, 4, 16).half(), s, -127, 127, 128)
    with pytest.raises(RuntimeError, match="elements"):
        ops.fakequant_per_channel(x.view(4, 16), torch.ones(3, device=DEV), -7, 7)
    with pytest.raises(RuntimeError, match="float32"):
        torch.ops.approxtorch.fakequant_per_tensor_claude.default(x.half(), s, -127, 127)
    with pytest.raises(RuntimeError, match="float32"):
        torch.ops.approxtorch.fakequant_per_tensor_backward_claude.default(x.half(), m, s)
    torch.cuda.synchronize()


def test_layers_reject_inputs_they_cannot_read():
    """Conv2d_int8 reads fp32 / fp16 / bf16 activations (fp64 is refused);
    Conv2d_uint8 reads fp32 only."""
    lut = t(perturbed_lut(1))
    l8 = at.nn.Conv2d_int8(3, 4, 3, lut, padding=1).to(DEV).train()
    with pytest.raises(RuntimeError, match="float32, float16 or bfloat16"):
        l8(torch.randn(1, 3, 5, 5, device=DEV).double())
    assert l8(torch.randn(1, 3, 5, 5, device=DEV).half()).dtype == torch.float32
    lu = at.nn.Conv2d_uint8(3, 4, 3, lut, padding=1).to(DEV).train()
    with pytest.raises(RuntimeError, match="float32"):
        lu(torch.randn(1, 3, 5, 5, device=DEV).to(torch.bfloat16))
    torch.cuda.synchronize()


# ---------------------------------------------- autograd and cache hazards
@pytest.mark.parametrize("grad", ["ste", "lre"])
def test_reuse_before_backward_raises_like_the_reference(grad):
    """The EMA updates scale_x / scale_w in place.  In the reference a layer
    run twice before backward makes the first call's backward fail with
    torch's in-place-modification error (its copy_() bumps the version);
    the HIP EMA must do the same instead of silently using the new scales."""
    lut_np = perturbed_lut(2)
    dx, dw = (t(a) for a in O.lre_tables(lut_np)) if grad == "lre" else (None, None)
    layer = at.nn.Conv2d_int8(4, 8, 3, t(lut_np), grad=grad, dx=dx, dw=dw, padding=1).to(DEV)
    layer.train()
    x1 = torch.randn(2, 4, 6, 6, device=DEV, requires_grad=True)
    y1 = layer(x1)
    layer(torch.randn(2, 4, 6, 6, device=DEV))
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        y1.sum().backward()
    # eval mode (frozen scales) has no hazard
    layer.eval()
    y3 = layer(x1)
    layer(x1)
    y3.sum().backward()


def test_uint8_reuse_before_backward_raises():
    layer = at.nn.Conv2d_uint8(3, 5, 3, t(asym_lut()), padding=1).to(DEV).train()
    y1 = layer(torch.randn(1, 3, 6, 6, device=DEV, requires_grad=True))
    layer(torch.randn(1, 3, 6, 6, device=DEV))
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        y1.sum().backward()


def test_lut_cache_distinguishes_views_of_one_storage():
    """Two views of one LUT storage with the same address, offset and version
    (the LUT and its transpose) must not share a cached image."""
    r = gen("lut_views")
    xi = r.integers(0, 256, (2, 17, 9), dtype=np.uint8)
    wv = r.integers(-128, 128, (7, 17)).astype(np.float32)
    lut = t(asym_lut())
    lutT = lut.view(256, 256).t()
    y0 = ops.bgemm_fake_int8_claude(t(xi), t(wv), lut)
    y1 = ops.bgemm_fake_int8_claude(t(xi), t(wv), lutT)
    wi = (wv + 128).astype(np.uint8)
    assert np.array_equal(y0.cpu().numpy().astype(np.int64), O.lut_gemm_i64(xi, wi, asym_lut()))
    lt = asym_lut().reshape(256, 256).T.reshape(-1)
    assert np.array_equal(y1.cpu().numpy().astype(np.int64), O.lut_gemm_i64(xi, wi, lt))


def test_lut_cache_survives_per_layer_copies():
    """A model moved with Module.to() holds one LUT copy per layer; every
    copy keeps its own cache entry, so repeated steps hit the cache."""
    lut_cpu = torch.from_numpy(perturbed_lut(4))
    layers = [at.nn.Conv2d_int8(2, 4, 1, lut_cpu) for _ in range(40)]
    model = torch.nn.Sequential(*layers).to(DEV).eval()
    ptrs = {m.lut.data_ptr() for m in model}
    assert len(ptrs) == 40
    x = torch.randn(1, 2, 4, 4, device=DEV)
    model[0].weight.data.fill_(0.0)
    with torch.no_grad():
        for m in model:
            m(x)
    before = len(ops._LUT_CACHE)
    with torch.no_grad():
        for m in model:
            m(x)
    assert len(ops._LUT_CACHE) == before
    assert all(ops._cache_key("image", m.lut, False) in ops._LUT_CACHE for m in model)
