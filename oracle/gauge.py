"""prompt_gauge_poly, restated from moge/model/v3.py:151-183 -- TEST INFRASTRUCTURE ONLY.

Per frame, a multiplicative correction exp(poly(u, v)) fitted robustly to log(prompt / prediction) on confident
prompt pixels, then applied at full resolution (infer's default `gauge_poly=2`, v3.py:841-853, model.py:77-100):

    ok = isfinite(depth) & depth > 0
    num = area(where(ok, depth, 0)), den = area(ok) at LiDAR resolution; z_lr = den > 0.5 ? num / max(den, 1e-6) : 0
    m = conf >= 2 & lidar > 0 & z_lr > 0 (conf None: 2 everywhere); fewer than 200 -> correction 1
    y = log(max(lidar, 1e-3)) - log(max(z_lr, 1e-3)); basis (1, u, v[, u^2, uv, v^2]) on linspace(-1, 1) grids
    w = 1; iters times: coef = lstsq(A w, y w); r = y - A coef; sc = 1.4826 median|r| + 1e-4 (the lower median);
                        w = min(2 sc / max(|r|, 1e-6), 1)
    non-finite coef -> correction 1; else exp(basis(U, V) coef) on the H x W grid

fp32 everywhere the reference computes in fp32; the least squares in fp64 (the reference: LAPACK on fp32), the
polynomial as a sequential fp32 sum over the basis terms.
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from .fit import area_pool
from .numerics import F32, exp_f32, log_f32

MIN_POINTS = 200


def linspace_f32(steps: int) -> np.ndarray:
    """torch.linspace(-1, 1, steps) in fp32 by its scalar rule: step = 2 / (steps - 1) in fp32; the first half
    start + step*i, the second half end - step*(steps-1-i). (torch's vectorised CPU loop may differ by an ulp.)"""
    if steps == 1:
        return np.float32([-1.0])
    step = F32(2.0) / F32(steps - 1)
    i = np.arange(steps)
    lo = F32(-1.0) + step * i.astype(np.float32)
    hi = F32(1.0) - step * (steps - 1 - i).astype(np.float32)
    return np.where(i < steps // 2, lo, hi).astype(np.float32)


def basis(u: np.ndarray, v: np.ndarray, degree: int) -> np.ndarray:
    """(1, u, v) or (1, u, v, u*u, u*v, v*v), last axis, fp32 (v3.py:164-168)."""
    cols = [np.ones_like(u), u, v]
    if degree >= 2:
        cols += [u * u, u * v, v * v]
    return np.stack(cols, -1).astype(np.float32)


def gauge_inputs(depth, lidar, conf):
    """z_lr, y, m at LiDAR resolution [B, h, w] (v3.py:155-159, 173-175)."""
    depth = np.asarray(depth, dtype=np.float32)
    B = depth.shape[0]
    h, w = np.shape(lidar)[-2:]
    ld = np.asarray(lidar, dtype=np.float32).reshape(B, h, w)
    cf = np.full_like(ld, 2.0) if conf is None else np.asarray(conf, dtype=np.float32).reshape(B, h, w)
    with np.errstate(invalid="ignore"):
        ok = np.isfinite(depth) & (depth > 0)
    num = area_pool(np.where(ok, depth, F32(0.0)), h, w)
    den = area_pool(ok.astype(np.float32), h, w)
    with np.errstate(divide="ignore", invalid="ignore"):
        z_lr = np.where(den > F32(0.5), num / np.maximum(den, F32(1e-6)), F32(0.0)).astype(np.float32)
    m = (cf >= F32(2.0)) & (ld > 0) & (z_lr > 0)
    y = (log_f32(np.maximum(ld, F32(1e-3))) - log_f32(np.maximum(z_lr, F32(1e-3)))).astype(np.float32)
    return z_lr, y, m


def poly_eval(A: np.ndarray, coef: np.ndarray) -> np.ndarray:
    """A @ coef as a sequential fp32 sum over the basis terms."""
    acc = np.zeros(A.shape[:-1], np.float32)
    for k in range(A.shape[-1]):
        acc = (acc + A[..., k] * F32(coef[k])).astype(np.float32)
    return acc


def fit_coef(A: np.ndarray, y: np.ndarray, iters: int = 3) -> np.ndarray:
    """The IRLS of v3.py:176-180 on the masked rows: returns the last lstsq solution (fp32)."""
    wgt = np.ones_like(y)
    coef = None
    for it in range(iters):
        Aw = (A * wgt[:, None]).astype(np.float32)
        yw = (y * wgt).astype(np.float32)
        coef = np.linalg.lstsq(Aw.astype(np.float64), yw.astype(np.float64), rcond=None)[0].astype(np.float32)
        r = (y - poly_eval(A, coef)).astype(np.float32)
        ar = np.abs(r)
        med = np.sort(ar)[(len(ar) - 1) // 2]  # torch.median: the lower of the two middle values
        sc = F32(1.4826) * med + F32(1e-4)
        with np.errstate(divide="ignore"):
            wgt = np.minimum((F32(2.0) * sc) / np.maximum(ar, F32(1e-6)), F32(1.0)).astype(np.float32)
    return coef


def gauge_poly(depth, lidar, conf: Optional[np.ndarray] = None, degree: int = 2, iters: int = 3,
               return_coef: bool = False):
    """[B, H, W] correction (v3.py:152-183); with return_coef also the per-frame coefficients (None: skipped)."""
    depth = np.asarray(depth, dtype=np.float32)
    B, H, W = depth.shape
    h, w = np.shape(lidar)[-2:]
    _, y, m = gauge_inputs(depth, lidar, conf)
    vv, uu = np.meshgrid(linspace_f32(h), linspace_f32(w), indexing="ij")
    Bm = basis(uu, vv, degree).reshape(h * w, -1)
    VV, UU = np.meshgrid(linspace_f32(H), linspace_f32(W), indexing="ij")
    Bf = basis(UU, VV, degree)
    out = np.ones((B, H, W), np.float32)
    coefs = []
    for b in range(B):
        mb = m[b].reshape(-1)
        if mb.sum() < MIN_POINTS:
            coefs.append(None)
            continue
        coef = fit_coef(Bm[mb], y[b].reshape(-1)[mb], iters)
        if not np.all(np.isfinite(coef)):
            coefs.append(None)
            continue
        coefs.append(coef)
        out[b] = exp_f32(poly_eval(Bf, coef))
    return (out, coefs) if return_coef else out
