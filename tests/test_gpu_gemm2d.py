"""GPU parity of the plain (torch.mm-layout) LUT GEMM ops
gemm_fake_{int8,uint8}_claude(_save) (csrc/claude/gemm.cu) against the int64
oracle, following the sections of csrc/claude/test_gemm_claude.py: both
orientations, GEMV edges, row-tile edges, strided / transposed / uint8
inputs, LUT classes, the _save contract, degenerate shapes, invalid inputs.

y[m,n] = sum_k lut[a_idx[m,k] * 256 + b_idx[k,n]] is checked bit-exactly (the
kernel sums int32 exactly; the float conversion of the oracle's int64 sum
rounds the same way); the fp32-fallback LUT against the oracle's fp32
ascending-k sum, also bit-exactly.
"""
import numpy as np
import pytest
import torch

from approxtorch_amd.backend import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t(a, dtype=None):
    return torch.as_tensor(np.ascontiguousarray(a), device=DEV, dtype=dtype)


def ref(a_idx, b_idx, lut):
    """[M,N] int64 oracle via lut_gemm_i64 (x = A^T as one image, w = B^T)."""
    return O.lut_gemm_i64(a_idx.T[None], b_idx.T, lut)[0].T


def perturbed(seed):
    r = np.random.default_rng(seed)
    a = np.arange(256) - 128
    p = a[:, None] * a[None, :]
    e = np.rint(r.normal(0, 1, p.shape) * (0.02 * np.abs(p) + 1))
    return np.clip(p + e, -32768, 32767).reshape(-1)


# (M, K, N): rows along N (M < N) and along M (M >= N), GEMV edges, tile edges
SHAPES = [(1, 1, 1), (1, 300, 77), (77, 300, 1), (2048, 64, 33), (2049, 65, 31),
          (31, 130, 2049), (500, 576, 500), (64, 1152, 4096), (5000, 96, 20), (3, 7, 5)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("signed", [True, False])
def test_gemm2d_matches_oracle(shape, signed):
    M, K, N = shape
    r = np.random.default_rng(M * 7919 + K * 31 + N + signed)
    a_idx = r.integers(0, 256, (M, K), dtype=np.uint8)
    b_idx = r.integers(0, 256, (K, N), dtype=np.uint8)
    lut = perturbed(M + N)
    off = 128 if signed else 0
    A = a_idx.astype(np.float32) - off
    B = b_idx.astype(np.float32) - off
    f = ops.gemm_fake_int8_claude if signed else ops.gemm_fake_uint8_claude
    y = f(t(A), t(B), t(lut, torch.float32)).cpu().numpy()
    assert y.shape == (M, N)
    assert np.array_equal(y, ref(a_idx, b_idx, lut).astype(np.float32))


def test_gemm2d_input_paths():
    """uint8 operands, a non-contiguous A, B as a transposed weight view
    W.t() (the Linear case), and fp32 values outside the index range (clamped)."""
    r = np.random.default_rng(5)
    M, K, N = 300, 200, 900
    lut = perturbed(5)
    lt = t(lut, torch.float32)
    a_idx = r.integers(0, 256, (M, K), dtype=np.uint8)
    w_idx = r.integers(0, 256, (N, K), dtype=np.uint8)
    want = ref(a_idx, w_idx.T, lut).astype(np.float32)
    # uint8 indices
    y = ops.gemm_fake_uint8_claude(t(a_idx), t(w_idx).t(), lt).cpu().numpy()
    assert np.array_equal(y, want)
    # non-contiguous A (transposed storage) and W.t() view, fp32 values
    At = t(a_idx.astype(np.float32).T).t()
    assert not At.is_contiguous()
    y = ops.gemm_fake_uint8_claude(At, t(w_idx.astype(np.float32)).t(), lt).cpu().numpy()
    assert np.array_equal(y, want)
    # the other orientation (M > N) with the same views
    y2 = ops.gemm_fake_uint8_claude(t(w_idx.astype(np.float32)), At.t(), lt).cpu().numpy()
    assert np.array_equal(y2, ref(w_idx, a_idx.T, lut).astype(np.float32))
    # fp32 values beyond [0, 255] clamp to the table's edge
    Ac = a_idx.astype(np.float32)
    Ac[0, :4] = [-7.0, 300.0, 255.4, -0.4]
    ac_idx = a_idx.copy()
    ac_idx[0, :4] = [0, 255, 255, 0]
    y = ops.gemm_fake_uint8_claude(t(Ac), t(w_idx).t(), lt).cpu().numpy()
    assert np.array_equal(y, ref(ac_idx, w_idx.T, lut).astype(np.float32))


@pytest.mark.parametrize("kind", ["u16_product", "fp32_fallback"])
def test_gemm2d_lut_classes(kind):
    r = np.random.default_rng(9)
    M, K, N = 129, 77, 2100
    a_idx = r.integers(0, 256, (M, K), dtype=np.uint8)
    b_idx = r.integers(0, 256, (K, N), dtype=np.uint8)
    v = np.arange(256)
    if kind == "u16_product":
        lut = (v[:, None] * v[None, :]).reshape(-1)                     # uint16 class
        y = ops.gemm_fake_uint8_claude(t(a_idx), t(b_idx), t(lut, torch.float32))
        assert np.array_equal(y.cpu().numpy(), ref(a_idx, b_idx, lut).astype(np.float32))
    else:
        lut = (r.standard_normal(65536) * 3.0).astype(np.float32)       # non-integer
        y = ops.gemm_fake_uint8_claude(t(a_idx), t(b_idx), t(lut)).cpu().numpy()
        want = O.lut_gemm_f32(a_idx.T[None], b_idx.T, lut)[0].T
        assert np.array_equal(y, want)


def test_gemm2d_save_contract():
    r = np.random.default_rng(11)
    M, K, N = 70, 90, 3000
    a_idx = r.integers(0, 256, (M, K), dtype=np.uint8)
    b_idx = r.integers(0, 256, (K, N), dtype=np.uint8)
    lut = t(perturbed(11), torch.float32)
    y, aq, bq = ops.gemm_fake_uint8_claude_save(t(a_idx.astype(np.float32)),
                                                t(b_idx.astype(np.float32)), lut)
    assert aq.shape == (M, K) and bq.shape == (N, K)
    assert np.array_equal(aq.cpu().numpy(), a_idx)
    assert np.array_equal(bq.cpu().numpy(), b_idx.T)
    assert torch.equal(y, ops.gemm_fake_uint8_claude(t(a_idx), t(b_idx), lut))
    A8 = t(a_idx)
    _, aq2, _ = ops.gemm_fake_uint8_claude_save(A8, t(b_idx), lut)
    assert aq2.data_ptr() == A8.data_ptr()
    # the M >= N orientation writes the same images
    y3, aq3, bq3 = ops.gemm_fake_int8_claude_save(t(b_idx.T.astype(np.float32) - 128),
                                                  t(a_idx.T.astype(np.float32) - 128), lut)
    assert np.array_equal(aq3.cpu().numpy(), b_idx.T)
    assert np.array_equal(bq3.cpu().numpy(), a_idx)


def test_gemm2d_degenerate_and_invalid():
    lut = t(perturbed(1), torch.float32)
    assert ops.gemm_fake_int8_claude(torch.zeros(0, 5, device=DEV),
                                     torch.zeros(5, 7, device=DEV), lut).shape == (0, 7)
    assert ops.gemm_fake_int8_claude(torch.zeros(4, 5, device=DEV),
                                     torch.zeros(5, 0, device=DEV), lut).shape == (4, 0)
    y = ops.gemm_fake_int8_claude(torch.zeros(4, 0, device=DEV), torch.zeros(0, 6, device=DEV),
                                  lut)
    assert y.shape == (4, 6) and torch.count_nonzero(y) == 0
    with pytest.raises(RuntimeError):
        ops.gemm_fake_int8_claude(torch.zeros(4, 5, device=DEV), torch.zeros(6, 7, device=DEV),
                                  lut)
    with pytest.raises(RuntimeError):
        ops.gemm_fake_int8_claude(torch.zeros(4, 5, device=DEV), torch.zeros(5, 7, device=DEV),
                                  lut[:100])
    with pytest.raises(RuntimeError):
        ops.gemm_fake_int8_claude(torch.zeros(2, 4, 5, device=DEV),
                                  torch.zeros(5, 7, device=DEV), lut)
    with pytest.raises(RuntimeError):
        ops.gemm_fake_int8_claude(torch.zeros(4, 5), torch.zeros(5, 7), lut.cpu())
