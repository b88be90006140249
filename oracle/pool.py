"""Sparse pooling and nearest upsampling, restated from the reference (test infrastructure only).

build_pool_cache (promptmoge/_fallback/flex_gemm/_core.py:339-395), perfect partition with output coordinates not
given; sparse_pool (_core.py:444-481); sparse_upsample (_core.py:484-505). NumPy, fp32 sums in input order (the
order of the reference's index_add_ on the CPU).
"""
from __future__ import annotations

from typing import Sequence, Tuple

import numpy as np

from .structure import linearise


def pool_cache(coords: np.ndarray, sparse_shape: Sequence[int], stride: Sequence[int],
               out_sparse_shape: Sequence[int]) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """build_pool_cache (_core.py:339-395) with kernel == stride, padding 0, output_coords None.
    coords (M, 4) int (b, x, y, z). Returns (out_coords (N, 4) int32, parent (M,) int32, seg_indices (M,) int32,
    seg_offsets (N + 1,) int64)."""
    coords = np.asarray(coords, dtype=np.int64)
    div = np.array([1] + [int(s) for s in stride], dtype=np.int64)
    down = np.floor_divide(coords, div[None, :])                           # _core.py:358-360
    keys = linearise(down, out_sparse_shape)                               # _core.py:367
    uniq, first, inverse = np.unique(keys, return_index=True, return_inverse=True)  # _core.py:370-375
    out_coords = down[first].astype(np.int32)
    order = np.argsort(inverse, kind="stable")                             # _core.py:385
    counts = np.bincount(inverse, minlength=uniq.shape[0])                 # _core.py:387
    offs = np.zeros(uniq.shape[0] + 1, dtype=np.int64)
    offs[1:] = np.cumsum(counts)                                           # _core.py:388-389
    return out_coords, inverse.astype(np.int32), order.astype(np.int32), offs


def sparse_pool(feats: np.ndarray, parent: np.ndarray, num_out: int, reduce: str = "mean") -> np.ndarray:
    """sparse_pool's reduction (_core.py:464-476): acc.index_add_(0, parent, feats), then / bincount for 'mean'."""
    feats = np.asarray(feats, dtype=np.float32)
    acc = np.zeros((num_out, feats.shape[1]), dtype=np.float32)
    np.add.at(acc, parent.astype(np.int64), feats)                         # sequential, in input order
    if reduce == "mean":
        counts = np.maximum(np.bincount(parent, minlength=num_out), 1).astype(np.float32)
        acc = acc / counts[:, None]
    elif reduce != "sum":
        raise NotImplementedError(reduce)
    return acc


def sparse_upsample(feats: np.ndarray, parent: np.ndarray) -> np.ndarray:
    """sparse_upsample 'nearest' (_core.py:500): feats.index_select(0, parent)."""
    return np.asarray(feats)[np.asarray(parent, dtype=np.int64)]
