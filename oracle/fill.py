"""nearest_fill (promptmoge/model.py:61-72), restated -- TEST INFRASTRUCTURE ONLY.

The reference fills missing LiDAR pixels (depth <= 0) from the index map of
scipy.ndimage.distance_transform_edt(~valid, return_indices=True) and sets their confidence to 1. That index map
is an exact Euclidean feature transform computed in two separable passes (axis 0, then axis 1); on equal
distances it keeps the valid pixel with the smallest column and, within that column, the smallest row. The
restatement below follows the same two passes:
  pass 1  per column, the nearest valid row (the upper one on ties);
  pass 2  per pixel, the least (F[i, c] - i)^2 + (j - c)^2 over columns c with a candidate, first minimum wins.
It is pinned against scipy itself (tests/test_oracle_fill.py), on random, structured and tie-heavy masks.
"""
from __future__ import annotations

import numpy as np


def column_rows(valid: np.ndarray) -> np.ndarray:
    """Pass 1: F[i, j] = nearest valid row of column j to row i (upper row on ties), -1 for an empty column."""
    valid = np.asarray(valid, dtype=bool)
    h = valid.shape[0]
    rows = np.arange(h)[:, None]
    far = 4 * h + 4
    up = np.maximum.accumulate(np.where(valid, rows, -far), axis=0)
    dn = np.minimum.accumulate(np.where(valid, rows, far)[::-1], axis=0)[::-1]
    F = np.where(rows - up <= dn - rows, up, dn)
    return np.where(np.abs(F) >= far, -1, F).astype(np.int64)


def nearest_index(valid: np.ndarray) -> np.ndarray:
    """(2, h, w) row/column of each pixel's nearest valid pixel, or -1 where the map has none."""
    valid = np.asarray(valid, dtype=bool)
    h, w = valid.shape
    F = column_rows(valid)
    out = np.full((2, h, w), -1, dtype=np.int64)
    cols = np.arange(w)
    for i in range(h):
        has = F[i] >= 0
        if not has.any():
            continue
        c = cols[has]
        d2 = (F[i, has] - i)[None, :] ** 2 + (cols[:, None] - c[None, :]) ** 2
        k = np.argmin(d2, axis=1)  # first minimum = smallest column
        out[0, i] = F[i, c[k]]
        out[1, i] = c[k]
    return out


def nearest_fill(depth: np.ndarray, conf: np.ndarray):
    """promptmoge.model.nearest_fill (model.py:61-72): the filled depth and confidence."""
    valid = depth > 0
    if valid.all() or not valid.any():
        return depth, conf
    idx = nearest_index(valid)
    return depth[idx[0], idx[1]], np.where(valid, conf, 1).astype(conf.dtype)
