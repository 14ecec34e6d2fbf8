"""Native backend: libatx.so (HIP, gfx950) behind a ctypes C ABI.

Importing this package loads the library and registers the reference's op
schemas under torch.ops.approxtorch (csrc/claude/bgemm_float_claude.cu:281-297,
bgemm_lre_backward_claude.cu:892-908, gemm.cu:292-307, dwconv_claude.cu:279-285,
quantization.cu:313-325, csrc/cuda/bgemm_custom_grad_optimize.cu:590-602),
implemented for the CUDA dispatch key (PyTorch-ROCm's key for GPU tensors)
only, as in the reference.
"""
import torch

from . import _lib, ops

_lib.load()


def _fp32_fq(x, s, qmin, qmax, z=None):
    # the reference's fused ops take fp32 x only (csrc/claude/quantization.cu:190-193)
    ops.require_cuda_f32(x, "x")
    return ops.fakequant_per_tensor(x, s, qmin, qmax, z)[:2]


def _fp32_fq_bwd(go, m, s):
    ops.require_cuda_f32(go, "grad_output")
    return ops.fakequant_per_tensor_backward(go, m, s)


_SCHEMAS = {
    "bgemm_fake_int8_forward_cuda_claude":
        ("(Tensor x, Tensor w, Tensor lut) -> Tensor", ops.bgemm_fake_int8_claude),
    "bgemm_fake_int8_forward_cuda_claude_cfg":
        ("(Tensor x, Tensor w, Tensor lut, int cfg) -> Tensor", ops.bgemm_fake_int8_claude_cfg),
    "bgemm_fake_int8_forward_cuda_claude_save":
        ("(Tensor x, Tensor w, Tensor lut) -> (Tensor, Tensor, Tensor)",
         ops.bgemm_fake_int8_claude_save),
    "bgemm_fake_uint8_forward_cuda_claude":
        ("(Tensor x, Tensor w, Tensor lut) -> Tensor", ops.bgemm_fake_uint8_claude),
    "bgemm_fake_uint8_forward_cuda_claude_cfg":
        ("(Tensor x, Tensor w, Tensor lut, int cfg) -> Tensor", ops.bgemm_fake_uint8_claude_cfg),
    "bgemm_fake_uint8_forward_cuda_claude_save":
        ("(Tensor x, Tensor w, Tensor lut) -> (Tensor, Tensor, Tensor)",
         ops.bgemm_fake_uint8_claude_save),
    "gemm_fake_int8_forward_cuda_claude":
        ("(Tensor A, Tensor B, Tensor lut) -> Tensor", ops.gemm_fake_int8_claude),
    "gemm_fake_int8_forward_cuda_claude_cfg":
        ("(Tensor A, Tensor B, Tensor lut, int cfg) -> Tensor", ops.gemm_fake_int8_claude_cfg),
    "gemm_fake_int8_forward_cuda_claude_save":
        ("(Tensor A, Tensor B, Tensor lut) -> (Tensor, Tensor, Tensor)",
         ops.gemm_fake_int8_claude_save),
    "gemm_fake_uint8_forward_cuda_claude":
        ("(Tensor A, Tensor B, Tensor lut) -> Tensor", ops.gemm_fake_uint8_claude),
    "gemm_fake_uint8_forward_cuda_claude_cfg":
        ("(Tensor A, Tensor B, Tensor lut, int cfg) -> Tensor", ops.gemm_fake_uint8_claude_cfg),
    "gemm_fake_uint8_forward_cuda_claude_save":
        ("(Tensor A, Tensor B, Tensor lut) -> (Tensor, Tensor, Tensor)",
         ops.gemm_fake_uint8_claude_save),
    "dwconv_fake_int8_claude":
        ("(Tensor x, Tensor w, Tensor lut, int kh, int kw, int sh, int sw, int ph, int pw, "
         "int dilh, int dilw) -> (Tensor, Tensor)",
         lambda x, w, lut, kh, kw, sh, sw, ph, pw, dh, dw: ops.dwconv_fake_int8_claude(
             x, w, lut, (kh, kw), (sh, sw), (ph, pw), (dh, dw))),
    "im2col_u8":
        ("(Tensor x, int kh, int kw, int sh, int sw, int ph, int pw, int dilh, int dilw) -> Tensor",
         lambda x, kh, kw, sh, sw, ph, pw, dh, dw: ops.im2col_u8(x, (kh, kw), (sh, sw), (ph, pw),
                                                                 (dh, dw))),
    "lut_map": ("(Tensor x, Tensor lut) -> Tensor", ops.lut_map),
    "lut_map_pad":
        ("(Tensor x, Tensor lut, int ph, int pw) -> Tensor",
         lambda x, lut, ph, pw: ops.lut_map_pad(x, lut, (ph, pw))),
    "bgemm_lre_backward_claude":
        ("(Tensor grad_output, Tensor x, Tensor w, Tensor dx, Tensor dw) -> (Tensor, Tensor)",
         ops.bgemm_lre_backward_claude),
    "bgemm_lre_backward_claude_cfg":
        ("(Tensor grad_output, Tensor x, Tensor w, Tensor dx, Tensor dw, int cfg) "
         "-> (Tensor, Tensor)", ops.bgemm_lre_backward_claude_cfg),
    "bgemm_lre_backward_claude_im2col":
        ("(Tensor grad_output, Tensor x, Tensor w, Tensor dx, Tensor dw, int kh, int kw, "
         "int sh, int sw, int ph, int pw, int dilh, int dilw) -> (Tensor, Tensor)",
         lambda go, x, w, dx, dw, kh, kw, sh, sw, ph, pw, dh, dwl:
             ops.bgemm_lre_backward_claude_im2col(go, x, w, dx, dw, (kh, kw), (sh, sw),
                                                  (ph, pw), (dh, dwl))),
    "bgemm_custom_grad_uint8_dx":
        ("(Tensor X, Tensor W, Tensor dY, Tensor dx_lut) -> Tensor",
         ops.bgemm_custom_grad_uint8_dx),
    "bgemm_custom_grad_uint8_dw":
        ("(Tensor X, Tensor W, Tensor dY, Tensor dw_lut) -> Tensor",
         ops.bgemm_custom_grad_uint8_dw),
    "bgemm_custom_grad_int8_dx":
        ("(Tensor X, Tensor W, Tensor dY, Tensor dx_lut) -> Tensor",
         ops.bgemm_custom_grad_int8_dx),
    "bgemm_custom_grad_int8_dw":
        ("(Tensor X, Tensor W, Tensor dY, Tensor dw_lut) -> Tensor",
         ops.bgemm_custom_grad_int8_dw),
    "fakequant_per_tensor_claude":
        ("(Tensor x, Tensor scale, int qmin, int qmax) -> (Tensor, Tensor)",
         lambda x, s, qmin, qmax: _fp32_fq(x, s, qmin, qmax)),
    "fakequant_per_tensor_backward_claude":
        ("(Tensor grad_output, Tensor mask, Tensor scale) -> Tensor",
         lambda go, m, s: _fp32_fq_bwd(go, m, s)),
    "fakequant_per_tensor_asymmetric_claude":
        ("(Tensor x, Tensor scale, Tensor zero_point, int qmin, int qmax) -> (Tensor, Tensor)",
         lambda x, s, z, qmin, qmax: _fp32_fq(x, s, qmin, qmax, z)),
    "fakequant_per_tensor_asymmetric_backward_claude":
        ("(Tensor grad_output, Tensor mask, Tensor scale) -> Tensor",
         lambda go, m, s: _fp32_fq_bwd(go, m, s)),
}


def _register():
    try:
        lib = torch.library.Library("approxtorch", "DEF")
    except RuntimeError:
        return None    # already registered in this process
    for name, (schema, fn) in _SCHEMAS.items():
        lib.define(name + schema)
        lib.impl(name, fn, "CUDA")
    return lib


_TORCH_LIBRARY = _register()
