"""GPU parity of sparse pooling and nearest upsampling (pmg_pool_cache / pmg_sparse_pool / pmg_sparse_upsample and the
flex_gemm shim's build_pool_cache, sparse_pool, sparse_upsample, SparsePool3d, SparseUpsample3d) against
oracle/pool.py (_core.py:339-505): cache arrays bit-exact, fp32 pooled features bit-exact (same summation order),
upsampled rows bit-exact."""
import numpy as np
import pytest
import torch

from oracle import pool as op
from oracle import structure as ost
from promptmoge_amd import flex_gemm as fg
from promptmoge_amd import ops, spec

from conftest import announce

pytestmark = pytest.mark.gpu


def _coords(rng, n, B, ext):
    b = rng.integers(0, B, n)
    xyz = np.stack([rng.integers(0, e, n) for e in ext], 1)
    c = np.unique(np.concatenate([b[:, None], xyz], 1), axis=0)
    return c[rng.permutation(len(c))].astype(np.int32)


def _check_cache(coords, shape, stride, gpu):
    osh = [shape[0]] + [-(-int(s) // int(k)) for s, k in zip(shape[1:], stride)]
    oc, parent, seg, offs = ops.pool_cache(torch.from_numpy(coords).to(gpu), shape, stride, osh)
    torch.cuda.synchronize()
    eoc, ep, es, eo = op.pool_cache(coords, shape, stride, osh)
    assert np.array_equal(oc.cpu().numpy(), eoc)
    assert np.array_equal(parent.cpu().numpy(), ep)
    assert np.array_equal(seg.cpu().numpy(), es)
    assert np.array_equal(offs.cpu().numpy(), eo)
    return oc, parent, seg, offs, ep


@pytest.mark.parametrize("n,B,ext,stride", [(20_000, 2, (40, 37, 65), (2, 2, 2)), (5_000, 1, (9, 300, 7), (2, 4, 1)),
                                            (1, 1, (3, 3, 3), (2, 2, 2)), (70_001, 3, (64, 64, 64), (2, 2, 2))])
def test_pool_cache_matches_oracle(gpu, n, B, ext, stride):
    announce(f"pool cache n={n} B={B} ext={ext} stride={stride}")
    rng = np.random.default_rng(n)
    coords = _coords(rng, n, B, ext)
    _check_cache(coords, (B, *ext), stride, gpu)


def test_pool_cache_level0_raster(gpu):
    """Model A's level-0 voxels (one per pixel, raster order) pooled by 2: the first U-Net level."""
    announce("pool cache level-0 raster 480x640")
    cfg = spec.CONFIGS["A"]
    sc = spec.make_scene(cfg)
    _, coords, Z, _ = ost.voxelize(sc.points[None])
    oc, parent, seg, offs, ep = _check_cache(coords.astype(np.int32), (1, cfg.H, cfg.W, Z), (2, 2, 2), gpu)
    assert oc.shape[0] == ep.max() + 1


def test_pool_cache_rejects_voxels_outside_the_grid(gpu):
    c = torch.tensor([[0, 1, 1, 1], [0, 5, 0, 0]], dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError):
        ops.pool_cache(c, (1, 4, 4, 4), (2, 2, 2), (1, 2, 2, 2))


@pytest.mark.parametrize("C", [4, 48, 13])
def test_sparse_pool_and_upsample_match_oracle(gpu, C):
    announce(f"sparse pool / upsample C={C}")
    rng = np.random.default_rng(C)
    coords = _coords(rng, 30_000, 2, (40, 41, 42))
    shape = torch.Size([2, 40, 41, 42, C])
    f = rng.normal(size=(len(coords), C)).astype(np.float32)
    ct = torch.from_numpy(coords).to(gpu)
    ft = torch.from_numpy(f).to(gpu)
    for reduce in ("mean", "sum"):
        pooled, oc, osh, cache = fg.ops.sparse_pool(ft, ct, shape, (2, 2, 2), reduce=reduce)
        eoc, ep, _, _ = op.pool_cache(coords, shape[:4], (2, 2, 2), list(osh[:4]))
        want = op.sparse_pool(f, ep, len(eoc), reduce)
        assert tuple(osh) == (2, 20, 21, 21, C)
        assert np.array_equal(oc.cpu().numpy(), eoc)
        assert np.array_equal(pooled.cpu().numpy(), want)
    up, uc, ush, _ = fg.ops.sparse_upsample(pooled, oc, osh, (2, 2, 2), output_coords=ct, output_shape=shape,
                                            neighbor_cache=cache.T)
    assert uc is ct and tuple(ush) == tuple(shape)
    assert np.array_equal(up.cpu().numpy(), op.sparse_upsample(want, ep))
    # the nn modules, as PoolDown / NearestUp call them (flex_sparse_blocks.py:78-105)
    p, u = fg.nn.SparsePool3d(2), fg.nn.SparseUpsample3d(2)
    pooled2, oc2, osh2, cache2 = p(ft, ct, shape, output_shape=osh)
    assert np.array_equal(pooled2.cpu().numpy(), op.sparse_pool(f, ep, len(eoc), "mean"))
    up2, _, _, _ = u(pooled2, oc2, osh2, output_coords=ct, output_shape=shape, neighbor_cache=cache2.T)
    assert np.array_equal(up2.cpu().numpy(), op.sparse_upsample(pooled2.cpu().numpy(), ep))


def test_upsample_fp16_rows(gpu):
    rng = np.random.default_rng(1)
    f = torch.from_numpy(rng.normal(size=(100, 24)).astype(np.float16)).to(gpu)
    parent = torch.from_numpy(rng.integers(0, 100, 1000).astype(np.int32)).to(gpu)
    out = ops.sparse_upsample(f, parent)
    assert torch.equal(out, f[parent.long()])
