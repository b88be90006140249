"""The flex_gemm plug-point package (promptmoge_amd.flex_gemm) mirrors the reference's fallback interface
(promptmoge/_fallback/flex_gemm: nn/__init__.py:20-110, ops/__init__.py:1-17, _core.py:65-82, 131-336, 399-441).

CPU tests check the interface (names, parameters, tap order, errors); GPU tests check the maps and convolutions
against the oracle: maps bit-exact, fp32 conv within 1e-5 of |out| (fp32 accumulation in another order than the
reference's per-tap loop), fp16 within 2e-3 relative of the fp32 oracle, bf16 within bf16 rounding."""
import importlib.util
import math
import sys

import numpy as np
import pytest
import torch

from oracle import conv as ocv
from oracle import structure as ost
from promptmoge_amd import flex_gemm as fg
from promptmoge_amd import spec

from conftest import announce


def test_install_makes_flex_gemm_importable():
    fg.install()
    assert importlib.util.find_spec("flex_gemm") is not None
    import flex_gemm
    from flex_gemm.nn import SparsePool3d, SparseUpsample3d, SubmanifoldConv3d  # noqa: F401
    from flex_gemm.ops import NeighborCache, build_submanifold_cache, submanifold_conv  # noqa: F401

    assert flex_gemm is fg and sys.modules["flex_gemm.nn"] is fg.nn


def test_kernel_delta_order_matches_oracle():
    d = fg.ops.make_conv_kernel_delta((3, 3, 3), (1, 1, 1), batch_dims=1).numpy()
    assert np.array_equal(d, ost.kernel_delta(1))
    d0 = fg.ops.make_conv_kernel_delta((3, 3, 3), (2, 2, 2)).numpy()
    assert d0.shape == (27, 3) and d0[0].tolist() == [-2, -2, -2] and d0[26].tolist() == [2, 2, 2]


def test_conv_module_parameters_and_init():
    torch.manual_seed(0)
    m = fg.nn.SubmanifoldConv3d(32, 48, 3)
    assert isinstance(m, fg.nn.SubmanifoldConv)
    assert m.weight.shape == (48, 3, 3, 3, 32) and m.bias.shape == (48,)
    assert m.kernel_size == (3, 3, 3) and m.dilation == (1, 1, 1)
    bound = 1.0 / math.sqrt(32 * 27)
    assert float(m.bias.detach().abs().max()) <= bound and float(m.weight.detach().abs().max()) <= bound + 1e-6
    assert fg.nn.SubmanifoldConv3d(8, 16, 3, bias=False).bias is None
    assert [n for n, _ in m.named_parameters()] == ["weight", "bias"]


def test_pool_and_upsample_modules_and_interface_errors():
    p = fg.nn.SparsePool3d(2)
    u = fg.nn.SparseUpsample3d(2)
    assert p.kernel_size == (2, 2, 2) and p.stride == (2, 2, 2) and p.reduce == "mean" and u.scale_factor == (2, 2, 2)
    coords = torch.zeros((1, 4), dtype=torch.int32)
    # the reference's assertions (_core.py:349-350, 490-494), raised before any device work
    with pytest.raises(AssertionError):
        fg.ops.build_pool_cache(coords, (1, 4, 4, 4), (2, 2, 2), (3, 3, 3), (0, 0, 0))
    with pytest.raises(AssertionError):
        fg.ops.build_pool_cache(coords, (1, 4, 4, 4), (2, 2, 2), (2, 2, 2), (1, 1, 1))
    with pytest.raises(NotImplementedError):
        fg.ops.build_pool_cache(coords, (1, 4, 4, 4), (2, 2, 2), (2, 2, 2), (0, 0, 0), output_coords=coords)
    with pytest.raises(NotImplementedError):
        fg.ops.sparse_pool(torch.zeros(1, 4), coords, torch.Size([1, 4, 4, 4, 4]), (2, 2, 2), reduce="max")
    with pytest.raises(AssertionError):
        fg.ops.sparse_upsample(torch.zeros(1, 4), coords, torch.Size([1, 2, 2, 2, 4]), (2, 2, 2),
                               output_coords=coords, neighbor_cache=None)
    with pytest.raises(ValueError):  # coords on the CPU: the library wants device tensors
        fg.ops.build_pool_cache(coords, (1, 4, 4, 4), (2, 2, 2), (2, 2, 2), (0, 0, 0))


def test_unsupported_kernels_rejected_before_any_device_work():
    coords = torch.zeros((1, 4), dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        fg.ops.build_submanifold_cache(coords, (1, 4, 4, 4), (5, 5, 5))
    with pytest.raises(NotImplementedError):
        fg.ops.build_submanifold_cache(coords, (1, 4, 4, 4), (3, 3, 3), dilation=(2, 2, 2))
    with pytest.raises(ValueError):
        fg.ops.build_submanifold_cache(coords, (1, 4, 4, 4), (3, 3, 3))  # coords on the CPU


def _level0(seed=3, B=2, H=40, W=56):
    cfg = spec.StepConfig("f", H, W, 40.0, 40.0, W / 2, H / 2, 16, 1, "int8", seed=seed)
    sc = spec.make_scene(cfg)
    pts = np.stack([sc.points] + [sc.points * np.float32(1.0 + 0.01 * b) for b in range(1, B)])
    zq, coords, Z, _ = ost.voxelize(pts)
    return coords.astype(np.int32), (B, H, W, Z)


@pytest.mark.gpu
def test_cache_level0_uses_column_stencil(gpu):
    announce("flex_gemm cache level 0")
    coords, shape = _level0()
    c = torch.from_numpy(coords).to(gpu)
    cache = fg.ops.build_submanifold_cache(c, shape, (3, 3, 3))
    assert cache.build_backend == "column" and cache.symmetric
    ref = ost.nmap_column(coords[:, 3].reshape(shape[:3]))
    assert np.array_equal(cache.nmap.cpu().numpy(), ref)
    assert np.array_equal(cache.tile_mask.cpu().numpy().view(np.uint32), ost.tile_masks(ref))
    occ = cache.occupancy()
    assert occ["V"] == 27 and occ["rows"] == coords.shape[0] and 1 <= occ["min"] and occ["max"] <= 9


@pytest.mark.gpu
def test_cache_generic_uses_hash(gpu):
    announce("flex_gemm cache generic")
    coords = spec.make_voxels(20_000, 64, seed=5).astype(np.int32)
    rng = np.random.default_rng(0)
    coords = coords[rng.permutation(coords.shape[0])]  # any order: the map indexes the caller's order
    shape = (1, 64, 64, 64)
    cache = fg.ops.build_submanifold_cache(torch.from_numpy(coords).to(gpu), shape, (3, 3, 3))
    assert cache.build_backend == "hash"
    assert np.array_equal(cache.nmap.cpu().numpy(), ost.nmap_sorted(coords, shape))


@pytest.mark.gpu
def test_cache_sorted_set_uses_column_runs(gpu):
    """A set in _linearise order takes the column-run map (the same map); backend "hash" forces the hash."""
    announce("flex_gemm cache sorted set")
    coords = spec.make_voxels(20_000, 64, seed=6).astype(np.int32)  # lexicographically sorted
    shape = (1, 64, 64, 64)
    ref = ost.nmap_sorted(coords, shape)
    cache = fg.ops.build_submanifold_cache(torch.from_numpy(coords).to(gpu), shape, (3, 3, 3))
    assert cache.build_backend == "sorted"
    assert np.array_equal(cache.nmap.cpu().numpy(), ref)
    forced = fg.ops.build_submanifold_cache(torch.from_numpy(coords).to(gpu), shape, (3, 3, 3), backend="hash")
    assert forced.build_backend == "hash"
    assert np.array_equal(forced.nmap.cpu().numpy(), ref)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,ci,co", [(torch.float32, 32, 48), (torch.float32, 6, 10), (torch.float16, 64, 64),
                                         (torch.bfloat16, 16, 32), (torch.float32, 64, 64), (torch.float16, 32, 32),
                                         (torch.float16, 128, 128), (torch.bfloat16, 64, 64)])
def test_submanifold_conv_matches_oracle(gpu, dtype, ci, co):
    announce(f"flex_gemm conv {dtype} {ci}->{co}")
    coords, shape = _level0(seed=ci + co)
    rng = np.random.default_rng(ci * co)
    M = coords.shape[0]
    x = rng.normal(0, 1, size=(M, ci)).astype(np.float32)
    w = rng.normal(0, 0.05, size=(co, 3, 3, 3, ci)).astype(np.float32)
    b = rng.normal(0, 0.05, size=(co,)).astype(np.float32)
    X = torch.from_numpy(x).to(gpu).to(dtype)
    Wt, Bt = torch.from_numpy(w).to(gpu).to(dtype), torch.from_numpy(b).to(gpu).to(dtype)
    xs = X.float().cpu().numpy()
    ws, bs = Wt.float().cpu().numpy(), Bt.float().cpu().numpy()
    nm = ost.nmap_column(coords[:, 3].reshape(shape[:3]))
    ref = ocv.conv_float(xs.astype(np.float64), nm, ws.astype(np.float64), bs.astype(np.float64), dtype=np.float64)
    C_ = torch.from_numpy(coords).to(gpu)
    full = torch.Size([*shape, ci])
    with torch.no_grad():
        out, cache = fg.ops.submanifold_conv(X, C_, full, Wt, Bt)
        assert out.dtype == dtype and out.shape == (M, co)
        got = out.float().cpu().numpy()
        scale = np.abs(ref).max()
        tol = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 8e-3}[dtype]
        assert np.abs(got - ref).max() <= tol * scale
        # the module gives the same result and reuses the cache
        m = fg.nn.SubmanifoldConv3d(ci, co, 3).to(gpu).to(dtype)
        m.weight.copy_(Wt)
        m.bias.copy_(Bt)
        out2, cache2 = m(X, C_, full, neighbor_cache=cache)
        assert cache2 is cache and torch.equal(out2, out)


@pytest.mark.gpu
def test_conv_refuses_gradients_and_stale_cache(gpu):
    announce("flex_gemm conv errors")
    coords, shape = _level0()
    C_ = torch.from_numpy(coords).to(gpu)
    m = fg.nn.SubmanifoldConv3d(8, 16, 3).to(gpu)
    X = torch.zeros((coords.shape[0], 8), device=gpu)
    full = torch.Size([*shape, 8])
    with pytest.raises(RuntimeError):
        m(X, C_, full)  # grad mode with trainable weights: inference-only kernels
    with torch.no_grad():
        _, cache = m(X, C_, full)
        with pytest.raises(AssertionError):
            m(X[:-1], C_[:-1], full, neighbor_cache=cache)
