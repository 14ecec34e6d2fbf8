"""LUT files and gradient tables: the native text parser against
numpy.loadtxt (CPU), and the device LRE / DATE generators against the numpy
implementations of grad_lut and against the oracle's restatement (GPU; DATE
bit-exact, LRE to the fp32 rounding of an fp64 slope)."""
import os

import numpy as np
import pytest
import torch

from approxtorch_amd import grad_lut, load_lut
from approxtorch_amd.backend import ops
from oracle import oracle as O


def write(path, text):
    with open(path, "w") as f:
        f.write(text)
    return path


def test_parser_matches_loadtxt_on_lut_files(tmp_path):
    a = np.arange(256) - 128
    lut = (a[:, None] * a[None, :]) // 3
    p = os.path.join(tmp_path, "lut.txt")
    np.savetxt(p, lut, fmt="%d")
    with open(p) as f:
        body = f.read()
    p2 = write(os.path.join(tmp_path, "lut2.txt"), "# header comment\n\n" +
               body.replace("\n", "  # row end\n", 3) + "\n\n")
    want = np.loadtxt(p, dtype=np.int32).reshape(-1)
    for path in (p, p2):
        got = load_lut.load_lut(path)
        assert got.dtype == torch.int32
        assert np.array_equal(got.numpy(), want)


def test_parser_float_tables_and_errors(tmp_path):
    r = np.random.default_rng(0)
    v = (r.standard_normal(256) * 3).astype(np.float32)
    pa = os.path.join(tmp_path, "a.txt")
    pb = os.path.join(tmp_path, "b.txt")
    np.savetxt(pa, v, fmt="%.4f")
    np.savetxt(pb, v)                               # numpy's default %.18e
    da, db = load_lut.load_lre_grad_lut(pa, pb)
    assert np.array_equal(da.numpy(), np.loadtxt(pa, dtype=np.float32))
    assert np.array_equal(db.numpy(), np.loadtxt(pb, dtype=np.float32))
    with pytest.raises(ValueError, match="cannot parse"):
        ops.parse_text_table(write(os.path.join(tmp_path, "bad.txt"), "1 2 x3\n"))
    with pytest.raises(ValueError, match="not an integer"):
        load_lut.load_lut(write(os.path.join(tmp_path, "frac.txt"), "1.5 " * 65536))
    with pytest.raises(ValueError, match="expected 65536"):
        load_lut.load_lut(write(os.path.join(tmp_path, "short.txt"), "1 " * 100))
    with pytest.raises(FileNotFoundError):
        load_lut.load_lut(os.path.join(tmp_path, "missing.txt"))


def _luts():
    r = np.random.default_rng(3)
    a = np.arange(256) - 128
    prod = a[:, None] * a[None, :]
    return {
        "perturbed": np.clip(prod + np.rint(r.normal(0, 1, prod.shape) *
                                             (0.02 * np.abs(prod) + 1)), -32768, 32767),
        "u8_masked": (np.arange(256)[:, None] * np.arange(256)[None, :]) & ~63,
        "random_float": r.standard_normal((256, 256)) * 500,
    }


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["perturbed", "u8_masked", "random_float"])
@pytest.mark.parametrize("qtype", ["int8", "uint8"])
def test_device_lre_tables(name, qtype):
    lut = _luts()[name].astype(np.float32)
    ga, gb = grad_lut.lre(torch.from_numpy(lut).cuda(), qtype)
    wa, wb = grad_lut.lre(lut, qtype)
    oa, ob = O.lre_tables(lut, qtype)
    for got, want in ((ga, wa), (gb, wb), (ga, oa), (gb, ob)):
        got = got.cpu().numpy()
        assert got.dtype == np.float32
        # both are an fp64 OLS slope rounded to fp32; the sums' order may move
        # the fp64 value by a few ulp, at most one fp32 ulp after rounding
        assert np.all(np.abs(got - want) <= np.spacing(np.abs(want)))


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["perturbed", "u8_masked", "random_float"])
@pytest.mark.parametrize("h", [0, 1, 2, 3, 4, 8, 32, 63, 100, 127])
def test_device_date_tables_bit_exact(name, h):
    lut = _luts()[name].astype(np.float32)
    ga, gb = grad_lut.DATE(torch.from_numpy(lut).cuda(), h)
    wa, wb = grad_lut.DATE(lut, h)
    assert np.array_equal(ga.cpu().numpy(), wa)
    assert np.array_equal(gb.cpu().numpy(), wb)
    # and directly against the oracle's loop restatement of grad_lut.py:39-142
    oa, ob = O.date_tables(lut, h)
    assert np.array_equal(ga.cpu().numpy(), oa)
    assert np.array_equal(gb.cpu().numpy(), ob)


@pytest.mark.gpu
def test_device_tables_are_cached_per_lut():
    lut = torch.from_numpy(_luts()["perturbed"].astype(np.float32)).cuda().view(-1)
    a1, _ = ops.date_tables(lut, 2)
    a2, _ = ops.date_tables(lut, 2)
    assert a1.data_ptr() == a2.data_ptr()
    lut.mul_(2)                                   # in-place update: new version, new tables
    a3, _ = ops.date_tables(lut, 2)
    assert a3.data_ptr() != a1.data_ptr()
    assert torch.equal(a3, 2 * a1)


@pytest.mark.parametrize("h", [1, 2, 4, 32, 100])
def test_date_smoothing_equals_per_slice_means(h):
    """grad_lut's vectorized smoothing equals the reference's formulation, a
    float32 `line[i-h:i+h+1].mean()` per position (grad_lut.py:39-60)."""
    lut = _luts()["random_float"].astype(np.float32)
    got = grad_lut._smooth(lut.copy(), h)
    for k in (0, 77, 255):
        line = lut[k]
        want = np.array([line[i - h:i + h + 1].mean() if h <= i <= 255 - h else line[i]
                         for i in range(256)], dtype=np.float32)
        assert np.array_equal(got[k], want)
