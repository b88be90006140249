"""Pins the oracle's submanifold convolution against an independent dense 3-D cross-correlation, and its int8
epilogues against closed forms."""
import numpy as np
import pytest

from oracle import conv as cv
from oracle import structure as st
from oracle.numerics import F32


def _sparse_set(rng, shape, frac):
    allc = np.stack(np.meshgrid(*[np.arange(s) for s in shape], indexing="ij"), -1).reshape(-1, 4)
    return allc[rng.random(allc.shape[0]) < frac]


@pytest.mark.parametrize("seed", range(3))
def test_int_accumulator_equals_dense_correlation(seed):
    rng = np.random.default_rng(seed)
    shape = (2, 6, 7, 8)
    coords = _sparse_set(rng, shape, 0.35)
    Ci, Co = 16, 32
    x = rng.integers(-127, 128, size=(coords.shape[0], Ci)).astype(np.int8)
    w = rng.integers(-127, 128, size=(Co, 3, 3, 3, Ci)).astype(np.int8)
    nm = st.nmap_sorted(coords, shape)
    acc = cv.conv_acc_int(x, nm, w)
    dense = cv.dense_correlation(coords, shape, x.astype(np.float64), w.astype(np.float64))
    assert np.array_equal(acc, dense.astype(np.int64))


def test_float_conv_equals_dense_correlation():
    rng = np.random.default_rng(5)
    shape = (1, 8, 8, 8)
    coords = _sparse_set(rng, shape, 0.3)
    x = rng.normal(size=(coords.shape[0], 24)).astype(np.float32)
    w = rng.normal(0, 0.05, size=(16, 3, 3, 3, 24)).astype(np.float32)
    b = rng.normal(size=16).astype(np.float32)
    nm = st.nmap_sorted(coords, shape)
    out = cv.conv_float(x, nm, w, b)
    ref = cv.dense_correlation(coords, shape, x.astype(np.float64), w.astype(np.float64)) + b
    assert np.abs(out - ref).max() < 1e-5


def test_epilogues_closed_form():
    acc = np.array([[100, -100, 0, 1 << 20]], dtype=np.int64)
    a, ws, b = F32(0.5), np.array([0.25, 0.25, 1.0, 1.0], np.float32), np.array([0.0, 1.0, -2.0, 0.0], np.float32)
    y = cv.dequant(acc, a, ws, b)
    assert y.tolist() == [[12.5, -11.5, -2.0, 524288.0]]
    r = cv.epilogue_r(acc, a, ws, b, np.ones((1, 4), np.float32))
    assert r.tolist() == [[13.5, -10.5, -1.0, 524289.0]]
    q = cv.epilogue_q(acc, a, ws, b, F32(8.0))  # multiplier 127/clip = 8
    silu = lambda v: v / (1 + np.exp(-v))
    expect = [int(np.clip(np.rint(silu(float(v)) * 8.0), -127, 127)) for v in y[0]]
    assert q.tolist()[0] == expect  # 12.5 -> 99.99..; -11.5 -> ~0; -2 -> -1.9 -> -2 (=-0.238/0.125); saturates


def test_conv_on_a_subset_of_rows():
    """A map of some rows (the sampled-row checks of large sets) gathers from all of x: the result is those rows
    of the full convolution, for the generic and the column-stencil map, integer and float."""
    rng = np.random.default_rng(4)
    z = rng.integers(0, 4, size=(1, 12, 14))
    nm = st.nmap_column(z)
    x = rng.integers(-127, 128, size=(nm.shape[0], 32)).astype(np.int8)
    w = rng.integers(-127, 128, size=(16, 3, 3, 3, 32)).astype(np.int8)
    rows = np.sort(rng.choice(nm.shape[0], 40, replace=False))
    full = cv.conv_acc_int(x, nm, w)
    assert np.array_equal(cv.conv_acc_int(x, nm[rows], w), full[rows])
    f = cv.conv_float(x.astype(np.float64), nm, w.astype(np.float64), dtype=np.float64)
    assert np.array_equal(cv.conv_float(x.astype(np.float64), nm[rows], w.astype(np.float64), dtype=np.float64),
                          f[rows])
    assert np.array_equal(f, full.astype(np.float64))
