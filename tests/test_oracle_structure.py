"""Pins the oracle's voxelisation and neighbour maps: closed-form rounding ties, raster order, brute force over a
coordinate dictionary, column == sorted backends (the reference's claimed cross-check, _core.py:27-32), and the
invariants of a submanifold map."""
import numpy as np
import pytest

from oracle import structure as st


def test_kernel_delta_order():
    d = st.kernel_delta()
    assert d.shape == (27, 4)
    assert d[13].tolist() == [0, 0, 0, 0]
    for v, (_, di, dj, dz) in enumerate(d.tolist()):
        assert v == (di + 1) * 9 + (dj + 1) * 3 + (dz + 1)


def test_voxelize_half_to_even_ties():
    # logz * 256 = k + 0.5 exactly: torch.round (and rint) rounds to even. Python's round() is half-to-even too.
    k = np.arange(-40, 40)
    logz = ((k + 0.5) / 256.0).astype(np.float32)
    pts = np.zeros((1, 1, k.size, 3), np.float32)
    pts[0, 0, :, 2] = logz
    zq, coords, Z, zmin = st.voxelize(pts)
    expect = np.array([round(float(v) * 256.0) for v in logz])
    assert zq.reshape(-1).tolist() == expect.tolist()
    assert zmin[0] == expect.min() and coords[:, 3].min() == 0 and Z == expect.max() - expect.min() + 1


def test_voxelize_raster_order_and_batches():
    rng = np.random.default_rng(1)
    pts = rng.normal(0.5, 0.3, size=(2, 5, 7, 3)).astype(np.float32)
    zq, coords, Z, zmin = st.voxelize(pts)
    b, i, j = np.meshgrid(np.arange(2), np.arange(5), np.arange(7), indexing="ij")
    assert np.array_equal(coords[:, 0], b.reshape(-1)) and np.array_equal(coords[:, 1], i.reshape(-1))
    assert np.array_equal(coords[:, 2], j.reshape(-1))
    for bb in range(2):
        zb = coords[coords[:, 0] == bb, 3]
        assert zb.min() == 0  # per-batch minimum (v3.py:333)
    assert Z == coords[:, 3].max() + 1


def _random_zmap(rng, B, H, W):
    # a random walk keeps neighbouring z within +-1 often, so most taps are exercised
    z = np.cumsum(rng.integers(-1, 2, size=(B, H, W)), axis=2) + np.cumsum(rng.integers(-1, 2, size=(B, H, 1)), axis=1)
    return z - z.min()


@pytest.mark.parametrize("seed", range(4))
def test_column_equals_bruteforce_and_sorted(seed):
    rng = np.random.default_rng(seed)
    B, H, W = 2, 7, 9
    z = _random_zmap(rng, B, H, W)
    b, i, j = np.meshgrid(np.arange(B), np.arange(H), np.arange(W), indexing="ij")
    coords = np.stack([b, i, j, z], -1).reshape(-1, 4)
    shape = (B, H, W, int(z.max()) + 1)
    col = st.nmap_column(z)
    assert np.array_equal(col, st.nmap_bruteforce(coords, shape))
    assert np.array_equal(col, st.nmap_sorted(coords, shape))


def test_column_invariants():
    rng = np.random.default_rng(7)
    z = _random_zmap(rng, 1, 60, 80)
    nm = st.nmap_column(z)
    M = nm.shape[0]
    assert np.array_equal(nm[:, 13], np.arange(M))                          # centre tap
    assert ((nm >= 0).sum(1) <= 9).all()                                    # one voxel per column, 9 columns
    o, v = np.nonzero(nm >= 0)
    assert np.array_equal(nm[nm[o, v], 26 - v], o)                          # symmetry
    zf = z.reshape(-1)
    dz = np.array([d[3] for d in st.kernel_delta()])
    assert np.array_equal(zf[nm[o, v]] - zf[o], dz[v])                      # the hit is at z + dz


@pytest.mark.parametrize("seed", range(3))
def test_sorted_equals_bruteforce_generic(seed):
    rng = np.random.default_rng(100 + seed)
    shape = (2, 6, 7, 8)
    allc = np.stack(np.meshgrid(*[np.arange(s) for s in shape], indexing="ij"), -1).reshape(-1, 4)
    coords = allc[rng.random(allc.shape[0]) < 0.3]
    coords = coords[rng.permutation(coords.shape[0])]  # the index refers to the caller's order
    assert np.array_equal(st.nmap_sorted(coords, shape), st.nmap_bruteforce(coords, shape))


def test_tile_masks_and_kmap():
    rng = np.random.default_rng(3)
    z = _random_zmap(rng, 1, 9, 11)  # M = 99, not a multiple of 16
    nm = st.nmap_column(z)
    tm = st.tile_masks(nm)
    for t in range(tm.size):
        exp = 0
        for r in range(16 * t, min(16 * t + 16, nm.shape[0])):
            for v in range(27):
                if nm[r, v] >= 0:
                    exp |= 1 << v
        assert int(tm[t]) == exp
    off, out_rows, in_rows = st.kmap_compact(nm)
    rebuilt = np.full_like(nm, -1)
    for v in range(27):
        rows = out_rows[off[v]:off[v + 1]]
        assert np.all(np.diff(rows) > 0)                                    # ascending, as nonzero() returns
        rebuilt[rows, v] = in_rows[off[v]:off[v + 1]]
    assert np.array_equal(rebuilt, nm)
