"""Trimmed least-squares scale/shift, restated from fit_scale_shift (moge/model/modules/prompt_stem.py:211-240).

    w = mask; s, t = 1, 0; ok = sum(w) >= min_points
    for it in 0..iters:
        n = max(sum w, 1); sx, sy, sxx, sxy = weighted sums; den = n*sxx - sx^2
        s' = (n*sxy - sx*sy) / max(den, 1e-12) if den > 1e-12 else 1; t' = (sy - s'*sx) / n;  keep if ok
        if it == iters: stop
        r = |s*z + t - target| / max(target, 1e-3) on mask, +inf elsewhere
        k = max(long((1 - trim) * count), min_points)  (fp32 product, truncated; count = mask.sum())
        thr = kthvalue(r, min(k, N));  w = mask & (r <= thr)

`fit_f64` keeps the weighted sums in fp64 (the GPU kernel's choice); `fit_f32` is the reference's literal fp32
form (sums in fp32). Both use the same fp32 residual expression ((s*z) + t) - target.
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, exp_f32


def _resid(s, t, z, tg, mask):
    """r = |s*z + t - target| / target.clamp_min(1e-3), +inf off the mask (prompt_stem.py:233-234)."""
    e = np.float32(s) * z
    e = e + np.float32(t)
    e = e - tg
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.abs(e) / np.maximum(tg, F32(1e-3))
    return np.where(mask, r, F32(np.inf)).astype(np.float32)


def _kth(r, kk):
    """torch.kthvalue(r, kk).values: the kk-th smallest, 1-indexed (prompt_stem.py:238)."""
    return np.partition(r, kk - 1)[kk - 1]


def _keep(mask, r, thr):
    """w = mask & (r <= thr) (prompt_stem.py:239): every residual tied with the threshold is kept."""
    return mask & (r <= thr)


def _fit_one(z, tg, mask, iters, trim, min_points, acc):
    N = z.shape[0]
    keep = np.float32(1.0 - trim)
    count = int(mask.sum())
    ok = count >= min_points
    k = max(int(keep * np.float32(count)), min_points)      # prompt_stem.py:237
    kk = min(k, N)                                           # prompt_stem.py:238
    s, t = F32(1.0), F32(0.0)
    w = mask.copy()
    thr = None
    for it in range(iters + 1):
        zz = z[w].astype(acc)
        tt = tg[w].astype(acc)
        n = acc(w.sum())
        sx, sy = zz.sum(dtype=acc), tt.sum(dtype=acc)
        sxx, sxy = (zz * zz).sum(dtype=acc), (zz * tt).sum(dtype=acc)
        nn = max(n, acc(1.0))
        den = nn * sxx - sx * sx
        sn = (nn * sxy - sx * sy) / max(den, acc(1e-12)) if den > 1e-12 else acc(1.0)
        tn = (sy - sn * sx) / nn
        if ok:
            s, t = F32(sn), F32(tn)
        if it == iters:
            break
        r = _resid(s, t, z, tg, mask)
        thr = _kth(r, kk)
        w = _keep(mask, r, thr)
    return s, t, dict(count=count, k=k, ok=ok, thr=thr)


def fit_f64(z, target, mask, iters=4, trim=0.2, min_points=32, return_info=False):
    """z, target: [B, N] fp32; mask: [B, N] bool -> s, t: [B] fp32 (sums in fp64)."""
    return _fit(z, target, mask, iters, trim, min_points, np.float64, return_info)


def fit_f32(z, target, mask, iters=4, trim=0.2, min_points=32, return_info=False):
    """The reference's fp32 sums."""
    return _fit(z, target, mask, iters, trim, min_points, np.float32, return_info)


def _fit(z, target, mask, iters, trim, min_points, acc, return_info):
    z = np.asarray(z, dtype=np.float32).reshape(np.shape(z)[0], -1)
    target = np.asarray(target, dtype=np.float32).reshape(z.shape)
    mask = np.asarray(mask, dtype=bool).reshape(z.shape)
    res = [_fit_one(z[b], target[b], mask[b], iters, trim, min_points, acc) for b in range(z.shape[0])]
    s = np.array([r[0] for r in res], dtype=np.float32)
    t = np.array([r[1] for r in res], dtype=np.float32)
    return (s, t, [r[2] for r in res]) if return_info else (s, t)


def nearest_index(dst: int, src: int) -> np.ndarray:
    """F.interpolate(mode='nearest') source index: min(floor(i * (src/dst)), src-1) with a float32 scale."""
    scale = np.float32(src) / np.float32(dst)
    return np.minimum(np.floor(np.arange(dst, dtype=np.float32) * scale).astype(np.int64), src - 1)


def prompt_inputs(points, lidar, conf):
    """_lidar_in_affine_frame's fit inputs (v3.py:373-378): z = exp(logz), target = nearest LiDAR, mask = valid &
    conf/2 >= 0.999. points [B, H, W, 3]; lidar, conf [B, dh, dw]. Returns z, target, mask [B, H*W], and (d, c)."""
    points = np.asarray(points, dtype=np.float32)
    B, H, W, _ = points.shape
    dh, dw = lidar.shape[-2:]
    iy, ix = nearest_index(H, dh), nearest_index(W, dw)
    d = np.asarray(lidar, dtype=np.float32)[:, iy][:, :, ix]
    c = np.clip(np.asarray(conf, dtype=np.float32)[:, iy][:, :, ix] / F32(2.0), F32(0.0), F32(1.0))
    valid = np.isfinite(d) & (d > 0)
    z = exp_f32(points[..., 2])
    mask = valid & (c >= F32(0.999))
    return z.reshape(B, -1), d.reshape(B, -1), mask.reshape(B, -1), d, c


def area_bounds(dst: int, src: int):
    """adaptive_avg_pool window of output index o: rows [floor(o*src/dst), ceil((o+1)*src/dst))."""
    o = np.arange(dst, dtype=np.int64)
    return (o * src) // dst, ((o + 1) * src + dst - 1) // dst


def area_pool(x, dh: int, dw: int) -> np.ndarray:
    """F.interpolate(x, (dh, dw), mode='area') for x [B, H, W] fp32: the window sum in fp32, row-major order, then
    divided by the window height and then by its width (adaptive_avg_pool2d)."""
    x = np.asarray(x, dtype=np.float32)
    B, H, W = x.shape
    r0, r1 = area_bounds(dh, H)
    c0, c1 = area_bounds(dw, W)
    out = np.empty((B, dh, dw), dtype=np.float32)
    for oh in range(dh):
        for ow in range(dw):
            win = x[:, r0[oh]:r1[oh], c0[ow]:c1[ow]].reshape(B, -1)
            s = np.zeros(B, dtype=np.float32)
            for k in range(win.shape[1]):
                s = (s + win[:, k]).astype(np.float32)
            out[:, oh, ow] = s / F32(r1[oh] - r0[oh]) / F32(c1[ow] - c0[ow])
    return out


def final_inputs(points, lidar, conf, mask_binary=None):
    """The final metric fit's inputs (v3.py:768-775) at LiDAR resolution: d_lr = area-pooled depth z = exp(logz);
    mask = conf >= 2 & lidar > 0 & d_lr > 0 (& area-pooled mask_binary > 0.99). Returns z, target, mask [B, dh*dw]."""
    points = np.asarray(points, dtype=np.float32)
    B = points.shape[0]
    lidar = np.asarray(lidar, dtype=np.float32).reshape(B, *np.shape(lidar)[-2:])
    conf = np.asarray(conf, dtype=np.float32).reshape(lidar.shape)
    dh, dw = lidar.shape[-2:]
    z = area_pool(exp_f32(points[..., 2]), dh, dw)
    mask = (conf >= F32(2.0)) & (lidar > 0) & (z > 0)
    if mask_binary is not None:
        mask &= area_pool(np.asarray(mask_binary, dtype=np.float32), dh, dw) > F32(0.99)
    return z.reshape(B, -1), lidar.reshape(B, -1), mask.reshape(B, -1)


def post_depth(points, st, mask=None):
    """post_depth (MetricFit.metal:200-211; v3.py:776): d = s * exp(logz) + t in fp32 per frame; +inf where the mask
    is false or d <= 0. points [B, H, W, 3], st (s [B], t [B]), mask [B, H, W] or None."""
    from .numerics import exp_f32

    logz = np.asarray(points, np.float32)[..., 2]
    s = np.asarray(st[0], np.float32).reshape(-1, 1, 1)
    t = np.asarray(st[1], np.float32).reshape(-1, 1, 1)
    d = (s * exp_f32(logz) + t).astype(np.float32)
    ok = d > 0
    if mask is not None:
        ok &= np.asarray(mask, bool)
    return np.where(ok, d, np.float32(np.inf)).astype(np.float32)
