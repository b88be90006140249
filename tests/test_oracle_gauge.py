"""The prompt gauge restatement (oracle/gauge.py, v3.py:152-183) pinned by torch's own linspace / median conventions
on the CPU and by closed-form recoveries: a LiDAR map that is exactly the pooled depth times exp(polynomial) gives
back that polynomial, also with gross outliers (IRLS), and too few points give the identity correction."""
import numpy as np
import pytest
import torch

from oracle import gauge as og
from oracle.fit import area_pool


@pytest.mark.parametrize("n", [1, 2, 3, 7, 8, 33, 64, 192, 256, 1008])
def test_linspace_matches_torch(n):
    ours = og.linspace_f32(n)
    ref = torch.linspace(-1, 1, n, dtype=torch.float32).numpy()
    assert ours[0] == ref[0] and ours[-1] == ref[-1]
    # torch's vectorised loop rounds with fused multiply-adds: within an ulp of the scalar rule (an ulp of 1 near 0)
    np.testing.assert_allclose(ours, ref, rtol=1.2e-7, atol=6e-8)


def test_lower_median_convention():
    x = torch.tensor([3.0, 1.0, 4.0, 2.0])
    assert torch.median(x).item() == np.sort(x.numpy())[(4 - 1) // 2] == 2.0


def _scene(B=2, H=48, W=64, h=24, w=32, degree=2, seed=0):
    rng = np.random.default_rng(seed)
    yy, xx = np.meshgrid(np.linspace(0, 1, H), np.linspace(0, 1, W), indexing="ij")
    depth = np.stack([(1.5 + 0.8 * xx + 0.4 * np.sin(3 * yy) + 0.1 * b) for b in range(B)]).astype(np.float32)
    coef = rng.normal(0, 0.05, (B, 6 if degree >= 2 else 3)).astype(np.float32)
    vv, uu = np.meshgrid(og.linspace_f32(h), og.linspace_f32(w), indexing="ij")
    A = og.basis(uu, vv, degree)
    pooled = area_pool(depth, h, w).astype(np.float64)
    lidar = np.stack([pooled[b] * np.exp(A.astype(np.float64) @ coef[b].astype(np.float64)) for b in range(B)])
    return depth, lidar.astype(np.float32), np.full((B, h, w), 2.0, np.float32), coef


@pytest.mark.parametrize("degree", [1, 2])
def test_recovers_exact_polynomial(degree):
    depth, lidar, conf, coef = _scene(degree=degree)
    out, coefs = og.gauge_poly(depth, lidar, conf, degree=degree, return_coef=True)
    for b in range(depth.shape[0]):
        np.testing.assert_allclose(coefs[b], coef[b], rtol=0, atol=2e-5)
    H, W = depth.shape[1:]
    VV, UU = np.meshgrid(og.linspace_f32(H), og.linspace_f32(W), indexing="ij")
    want = np.exp(og.basis(UU, VV, degree).astype(np.float64) @ coef.T.astype(np.float64)).transpose(2, 0, 1)
    np.testing.assert_allclose(out, want, rtol=3e-5)


def test_irls_ignores_gross_outliers():
    depth, lidar, conf, coef = _scene(seed=3)
    rng = np.random.default_rng(4)
    bad = rng.random(lidar.shape) < 0.1
    lidar = np.where(bad, lidar * np.float32(1.6), lidar).astype(np.float32)
    _, coefs = og.gauge_poly(depth, lidar, conf, return_coef=True)
    for b in range(depth.shape[0]):
        np.testing.assert_allclose(coefs[b], coef[b], rtol=0, atol=1e-3)
    # one plain least-squares solve would be pulled far off by the same outliers
    _, one = og.gauge_poly(depth, lidar, conf, iters=1, return_coef=True)
    assert np.abs(one[0] - coef[0]).max() > 1e-2


def test_too_few_points_and_no_conf():
    depth, lidar, conf, coef = _scene(B=1)
    few = np.zeros_like(conf)
    few[0, :5, :5] = 2.0  # 25 confident pixels < 200
    np.testing.assert_array_equal(og.gauge_poly(depth, lidar, few), np.ones_like(depth))
    # conf None counts every pixel as confident
    np.testing.assert_allclose(og.gauge_poly(depth, lidar, None), og.gauge_poly(depth, lidar, conf), rtol=0, atol=0)
    # invalid depth is excluded from the pooled prediction (z_lr from the valid part of each window only)
    d2 = depth.copy()
    d2[0, 0, 0] = np.inf
    _, y, m = og.gauge_inputs(d2, lidar, conf)
    assert m[0, 0, 0] and np.isfinite(y[0, 0, 0])
