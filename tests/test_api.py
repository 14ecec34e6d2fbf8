"""Host-side API tests (CPU): convert_model (the reference's own unittest cases,
tests/test_convert_model.py:13-114), layer construction rules, state_dict
compatibility, LUT / gradient-table files, and the product path's refusal to
run on CPU tensors."""
import inspect

import numpy as np
import pytest
import torch
import torch.nn as nn

import approxtorch_amd as at
from approxtorch_amd.convert_model import convert_model
from approxtorch_amd.nn import Conv2d_int8, Conv2d_uint8
from approxtorch_amd.nn.Conv2d_uint8 import uint8_qparams
from oracle import oracle as O

LUT = torch.zeros(256, 256, dtype=torch.float32)


def test_public_api_has_only_unified_entry():
    params = inspect.signature(convert_model).parameters
    assert "x_quantizer" not in params and "w_quantizer" not in params
    assert not hasattr(at, "to_qat_int8")
    for name in ("lut", "grad", "dx", "dw", "bias", "stride", "padding", "dilation", "groups",
                 "update_scale", "scale_momentum", "weight_bits"):
        assert name in inspect.signature(Conv2d_int8).parameters


def test_int8_conversion_preserves_state_and_skips_first_conv():
    model = nn.Sequential(nn.Conv2d(3, 4, 3, padding=1),
                          nn.Sequential(nn.ReLU(), nn.Conv2d(4, 5, 1)))
    source = model[1][1]
    source.weight.requires_grad_(False)
    w0, b0 = source.weight.detach().clone(), source.bias.detach().clone()
    model.eval()
    result = convert_model(model, LUT, qtype="int8", weight_bits=5)
    assert result is model
    assert isinstance(model[0], nn.Conv2d)
    conv = model[1][1]
    assert isinstance(conv, Conv2d_int8)
    torch.testing.assert_close(conv.weight, w0)
    torch.testing.assert_close(conv.bias, b0)
    assert not conv.weight.requires_grad and not conv.training and conv.weight_bits == 5
    torch.testing.assert_close(conv.scale_w, w0.abs().amax(dim=(1, 2, 3)) / 15)


def test_uint8_conversion_initializes_weight_qparams():
    model = nn.Sequential(nn.Conv2d(2, 3, 3, bias=False))
    w0 = model[0].weight.detach().clone()
    convert_model(model, LUT, qtype="uint8", ignore_first_conv=False, update_scale=False)
    conv = model[0]
    assert isinstance(conv, Conv2d_uint8) and conv.bias is None and not conv.update_scale
    mn, mx = w0.amin(dim=(1, 2, 3)), w0.amax(dim=(1, 2, 3))
    s, z = uint8_qparams(mn, mx)
    torch.testing.assert_close(conv.w_min, mn)
    torch.testing.assert_close(conv.w_max, mx)
    torch.testing.assert_close(conv.scale_w, s)
    torch.testing.assert_close(conv.zero_w, z)


def test_root_conv_is_returned_as_replacement():
    src = nn.Conv2d(3, 4, 1)
    conv = convert_model(src, LUT, qtype="int8", ignore_first_conv=False)
    assert isinstance(conv, Conv2d_int8)
    torch.testing.assert_close(conv.weight, src.weight)


def test_unsupported_uint8_group_does_not_partially_convert():
    model = nn.Sequential(nn.Conv2d(4, 4, 1), nn.Conv2d(4, 4, 3, padding=1, groups=2))
    with pytest.raises(NotImplementedError):
        convert_model(model, LUT, qtype="uint8", ignore_first_conv=False)
    assert isinstance(model[0], nn.Conv2d) and isinstance(model[1], nn.Conv2d)


def test_invalid_arguments_fail_early():
    model = nn.Sequential(nn.Conv2d(1, 1, 1))
    with pytest.raises(ValueError, match="qtype"):
        convert_model(model, LUT, qtype="int4")
    with pytest.raises(ValueError, match="65536"):
        convert_model(model, torch.zeros(10))
    with pytest.raises(ValueError, match="weight_bits"):
        convert_model(model, LUT, weight_bits=9)
    with pytest.raises(TypeError, match="weight_bits"):
        convert_model(model, LUT, weight_bits=True)
    with pytest.raises(ValueError, match="grad"):
        Conv2d_int8(1, 1, 1, LUT, grad="bogus")
    with pytest.raises(ValueError, match="required"):
        Conv2d_int8(1, 1, 1, LUT, grad="lre")
    with pytest.raises(ValueError, match="65536"):
        Conv2d_int8(1, 1, 1, LUT, grad="custom", dx=torch.zeros(3), dw=torch.zeros(3))
    with pytest.raises(NotImplementedError):
        convert_model(nn.Sequential(nn.Conv2d(2, 2, 3, padding="same")), LUT,
                      ignore_first_conv=False)


def test_uint8_legacy_state_dict_and_zero_point_validation():
    a = Conv2d_uint8(2, 3, 3, LUT)
    sd = {k: v for k, v in a.state_dict().items()
          if k not in ("scale_x", "zero_x", "scale_w", "zero_w")}
    sd["x_min"] = torch.tensor(-2.0)
    sd["x_max"] = torch.tensor(6.0)
    b = Conv2d_uint8(2, 3, 3, LUT)
    b.load_state_dict(sd)                      # legacy min/max-only checkpoint
    s, z = uint8_qparams(torch.tensor(-2.0), torch.tensor(6.0))
    torch.testing.assert_close(b.scale_x, s)
    torch.testing.assert_close(b.zero_x, z)
    bad = a.state_dict()
    bad["zero_x"] = torch.tensor(3.5)
    with pytest.raises(RuntimeError, match="zero_x"):
        Conv2d_uint8(2, 3, 3, LUT).load_state_dict(bad)


def test_product_path_refuses_cpu_tensors():
    conv = Conv2d_int8(2, 3, 3, LUT)
    with pytest.raises(RuntimeError, match="CUDA"):
        conv(torch.randn(1, 2, 5, 5))


def test_load_lut_and_table_files(tmp_path):
    a = np.arange(256) - 128
    tbl = (a[:, None] * a[None, :])
    p = tmp_path / "mul8s.txt"
    np.savetxt(p, tbl, fmt="%d")
    lut = at.load_lut.load_lut(str(p))
    assert lut.dtype == torch.int32 and lut.shape == (65536,)
    assert torch.equal(lut, torch.from_numpy(tbl.reshape(-1)).int())
    ga, gb = at.grad_lut.lre(str(p), "int8", save_path=str(tmp_path / "m"))
    assert np.allclose(ga, a) and np.allclose(gb, a)
    da, db = at.load_lut.load_lre_grad_lut(str(tmp_path / "m_lre_grad_a.txt"),
                                           str(tmp_path / "m_lre_grad_b.txt"))
    assert torch.allclose(da, torch.from_numpy(a).float())


def test_grad_lut_date_matches_oracle_loops():
    rng = np.random.default_rng(3)
    lut = rng.integers(-3000, 3000, (256, 256)).astype(np.float32)
    for h in (1, 2, 32):
        ga, gb = at.grad_lut.DATE(lut, h)
        oa, ob = O.date_tables(lut, h)
        assert np.array_equal(ga, oa) and np.array_equal(gb, ob)


def test_grad_lut_lre_matches_oracle():
    rng = np.random.default_rng(4)
    lut = rng.integers(-3000, 3000, (256, 256)).astype(np.float32)
    for q in ("int8", "uint8"):
        ga, gb = at.grad_lut.lre(lut, q)
        oa, ob = O.lre_tables(lut, q)
        assert np.allclose(ga, oa, rtol=1e-6, atol=1e-6)
        assert np.allclose(gb, ob, rtol=1e-6, atol=1e-6)


def test_cpu_baseline_restatement_matches_oracle():
    from oracle import torch_cpu
    rng = np.random.default_rng(5)
    lut = rng.integers(-3000, 3000, 65536).astype(np.float32)
    ga, gb = O.lre_tables(lut)
    conv = Conv2d_int8(3, 6, 3, torch.from_numpy(lut), grad="lre", dx=torch.from_numpy(ga),
                       dw=torch.from_numpy(gb), bias=True, padding=1, stride=2)
    conv.scale_x.fill_(0.02)
    cpu = torch_cpu.LUTConv2dCPU(conv).eval()
    x = torch.randn(2, 3, 9, 8)
    xr = x.clone().requires_grad_()
    y = cpu(xr)
    want, ctx = O.conv_int8_forward(x.numpy(), conv.weight.detach().numpy(),
                                    conv.bias.detach().numpy(), lut, np.float32(0.02),
                                    conv.scale_w.numpy(), (3, 3), (2, 2), (1, 1), (1, 1))
    np.testing.assert_allclose(y.detach().double().numpy(), want, rtol=1e-5, atol=1e-3)
    go = torch.randn_like(y)
    y.backward(go)
    gx, gw, _ = O.conv_int8_backward(go.numpy(), ctx, np.float32(0.02), conv.scale_w.numpy(),
                                     "lre", (ga, gb), (3, 3), (2, 2), (1, 1), (1, 1))
    np.testing.assert_allclose(xr.grad.double().numpy(), gx, rtol=1e-4, atol=1e-3)


def test_conversion_walk_matches_named_modules_order_and_dedup():
    """Sites come in named_modules() order with shared modules once; a conv
    reachable by two paths is replaced at the first path only (as a
    named_modules-driven conversion would)."""
    from approxtorch_amd.convert_model import _conv_sites
    shared = nn.Conv2d(4, 4, 1)
    inner = nn.Sequential(nn.Conv2d(4, 4, 3, padding=1), shared)
    model = nn.Sequential(nn.Conv2d(3, 4, 1), inner, nn.ReLU(), shared, inner,
                          nn.ModuleDict({"a": nn.Conv2d(4, 2, 1)}))
    want = [id(m) for _, m in model.named_modules() if isinstance(m, nn.Conv2d)]
    assert [id(c) for _, _, c in _conv_sites(model)] == want
    convert_model(model, LUT, qtype="int8")
    assert isinstance(model[0], nn.Conv2d)                 # first conv skipped
    assert isinstance(inner[0], Conv2d_int8) and isinstance(inner[1], Conv2d_int8)
    assert model[3] is shared                              # second path untouched
    assert isinstance(model[5]["a"], Conv2d_int8)
    assert model[4] is inner


def test_custom_grad_schemas_name_their_tables_as_the_reference():
    """bgemm_custom_grad_optimize.cu:591-594 declares dx_lut / dw_lut, so
    keyword calls through torch.ops.approxtorch work unchanged."""
    for kind in ("uint8", "int8"):
        for d in ("dx", "dw"):
            op = getattr(torch.ops.approxtorch, f"bgemm_custom_grad_{kind}_{d}").default
            assert [a.name for a in op._schema.arguments] == ["X", "W", "dY", f"{d}_lut"]
