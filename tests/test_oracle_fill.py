"""Pins oracle/fill.py (nearest_fill, promptmoge/model.py:61-72) against scipy.ndimage's exact EDT index map --
the routine the reference calls -- on random, structured and tie-heavy masks."""
import numpy as np
import pytest

from oracle import fill

ndimage = pytest.importorskip("scipy.ndimage")


def _scipy_index(valid):
    return ndimage.distance_transform_edt(~valid, return_distances=False, return_indices=True)


def _masks():
    rng = np.random.default_rng(7)
    for _ in range(60):
        h, w = rng.integers(1, 40, 2)
        yield rng.random((h, w)) < rng.choice([0.02, 0.1, 0.5, 0.9])
    # tie-heavy lattices: every hole pixel has several equidistant sources
    for step in (2, 3, 4, 7):
        m = np.zeros((29, 31), bool)
        m[::step, ::step] = True
        yield m
        yield m.T.copy()
    m = np.zeros((20, 20), bool); m[0, 0] = m[19, 19] = True; yield m   # diagonal symmetry
    m = np.zeros((15, 40), bool); m[:, 5] = m[:, 34] = True; yield m    # two vertical lines
    m = np.zeros((40, 15), bool); m[5] = m[34] = True; yield m          # two horizontal lines
    m = np.ones((30, 30), bool); m[5:25, 5:25] = False; yield m         # one large hole
    m = np.zeros((1, 50), bool); m[0, [3, 9, 10, 40]] = True; yield m   # single row
    m = np.zeros((50, 1), bool); m[[0, 20, 22], 0] = True; yield m      # single column


def test_index_matches_scipy():
    for valid in _masks():
        if not valid.any():
            continue
        got = fill.nearest_index(valid)
        np.testing.assert_array_equal(got, _scipy_index(valid))


def test_column_pass_prefers_upper_row():
    valid = np.zeros((5, 1), bool)
    valid[[0, 4], 0] = True
    assert fill.column_rows(valid)[:, 0].tolist() == [0, 0, 0, 4, 4]


def test_fill_values_and_conf():
    rng = np.random.default_rng(3)
    depth = rng.uniform(0.5, 5.0, (33, 47)).astype(np.float32)
    depth[rng.random(depth.shape) < 0.3] = 0.0
    depth[1, 1] = np.nan
    conf = rng.integers(0, 3, depth.shape).astype(np.uint8)
    d, c = fill.nearest_fill(depth, conf)
    valid = depth > 0
    idx = _scipy_index(valid)
    np.testing.assert_array_equal(d, depth[tuple(idx)])
    np.testing.assert_array_equal(c, np.where(valid, conf, 1).astype(np.uint8))
    assert c.dtype == np.uint8 and (d > 0).all()


def test_fill_no_op_cases():
    d = np.ones((4, 5), np.float32)
    c = np.zeros((4, 5), np.float32)
    assert fill.nearest_fill(d, c)[0] is d
    z = np.zeros((4, 5), np.float32)
    assert fill.nearest_fill(z, c)[0] is z
