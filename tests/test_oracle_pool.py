"""Pins oracle/pool.py (build_pool_cache / sparse_pool / sparse_upsample, _core.py:339-505).

The reference's own code is not imported; the checks are torch's CPU library routines that the reference calls
(torch.unique(sorted=True, return_inverse=True), stable argsort, bincount, index_add_ and index_select on the CPU,
the same ops _core.py:339-505 is written with), a hand-checked small case, and invariants that a wrong index, a
dropped term or an unstable order would break."""
import numpy as np
import pytest
import torch

from oracle import pool as op
from oracle.structure import linearise


def _coords(rng, n, B=2, ext=(20, 17, 33)):
    b = rng.integers(0, B, n)
    xyz = np.stack([rng.integers(0, e, n) for e in ext], 1)
    c = np.unique(np.concatenate([b[:, None], xyz], 1), axis=0)
    return c[rng.permutation(len(c))].astype(np.int32)  # unique voxels in a random order


def _out_shape(shape, stride):
    return [shape[0]] + [-(-int(s) // int(k)) for s, k in zip(shape[1:], stride)]


def test_pool_cache_small_hand_case():
    # two voxels in one 2x2x2 cell, one in another; output keys sorted, parent/seg by input order
    c = np.array([[0, 3, 1, 1], [0, 0, 0, 1], [0, 1, 1, 0]], dtype=np.int32)
    oc, parent, seg, offs = op.pool_cache(c, (1, 4, 2, 2), (2, 2, 2), (1, 2, 1, 1))
    assert oc.tolist() == [[0, 0, 0, 0], [0, 1, 0, 0]]
    assert parent.tolist() == [1, 0, 0]
    assert seg.tolist() == [1, 2, 0]
    assert offs.tolist() == [0, 2, 3]


@pytest.mark.parametrize("stride", [(2, 2, 2), (2, 3, 4)])
def test_pool_cache_matches_torch_ops(stride):
    rng = np.random.default_rng(7)
    c = _coords(rng, 3000)
    shape = (2, 20, 17, 33)
    osh = _out_shape(shape, stride)
    oc, parent, seg, offs = op.pool_cache(c, shape, stride, osh)
    # the reference's op sequence with torch on the CPU (_core.py:358-389)
    t = torch.from_numpy(c.astype(np.int64))
    div = torch.tensor([1, *stride])
    down = torch.div(t, div.view(1, -1), rounding_mode="floor")
    keys = torch.from_numpy(linearise(down.numpy(), osh))
    uniq, inv = torch.unique(keys, sorted=True, return_inverse=True)
    first = torch.full((uniq.shape[0],), -1, dtype=torch.int64)
    first.scatter_reduce_(0, inv, torch.arange(down.shape[0]), reduce="amin", include_self=False)
    assert np.array_equal(oc, down[first].numpy())
    assert np.array_equal(parent, inv.numpy())
    assert np.array_equal(seg, torch.argsort(inv, stable=True).numpy())
    cnt = torch.bincount(inv, minlength=uniq.shape[0])
    assert np.array_equal(offs[1:], torch.cumsum(cnt, 0).numpy()) and offs[0] == 0
    # invariants: every member floors to its parent's coordinates; groups are in input order
    assert np.array_equal(np.floor_divide(c, np.array([1, *stride])), oc[parent])
    for r in range(len(oc)):
        g = seg[offs[r]:offs[r + 1]]
        assert np.all(np.diff(g) > 0) and np.all(parent[g] == r)


def test_sparse_pool_and_upsample_match_torch_ops():
    rng = np.random.default_rng(3)
    c = _coords(rng, 2000)
    oc, parent, seg, offs = op.pool_cache(c, (2, 20, 17, 33), (2, 2, 2), (2, 10, 9, 17))
    f = rng.normal(size=(len(c), 12)).astype(np.float32)
    n = len(oc)
    for reduce in ("mean", "sum"):
        got = op.sparse_pool(f, parent, n, reduce)
        acc = torch.zeros((n, 12))
        acc.index_add_(0, torch.from_numpy(parent.astype(np.int64)), torch.from_numpy(f))
        if reduce == "mean":
            acc = acc / torch.bincount(torch.from_numpy(parent.astype(np.int64)), minlength=n).clamp(min=1).float()[:, None]
        assert np.array_equal(got, acc.numpy())
    up = op.sparse_upsample(got, parent)
    assert np.array_equal(up, torch.from_numpy(got).index_select(0, torch.from_numpy(parent.astype(np.int64))).numpy())
