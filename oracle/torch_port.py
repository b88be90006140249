"""The reference's CPU path for one int8 refiner step, in torch on the host: the CPU baseline that bench.py times.

TEST / BASELINE INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and tests/). A restatement of the _fallback path
op for op with torch's CPU kernels, so that the baseline is the reference's algorithm on the host's cores (the
reference's own Python does not travel to the GPU box):

  prompt fit      fit_scale_shift (moge/model/modules/prompt_stem.py:211-240): masked sums, torch.kthvalue per batch
                  item, iters + 1 solves
  prompt feats    _lidar_in_affine_frame (v3.py:371-383) and the [residual, gate] stack (v3.py:552-554)
  voxelise        _voxelize (v3.py:327-340): torch.round(logz * 256), per-batch min
  neighbour map   _build_submanifold_nmap_column (promptmoge/_fallback/flex_gemm/_core.py:269-295)
  blocks          SparseResBlock3d (flex_sparse_blocks.py:70-75) under QAT fake quantisation (qat.py:28-57, 89-106),
                  each conv the _fallback submanifold_conv (_core.py:399-441): bias, then per tap the valid rows
                  (nonzero), index_select, mm, index_add_
  output          out_proj, logz + out (v3.py:356-359)
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

QMAX = 127.0


def fit_scale_shift(z, target, mask, iters=4, trim=0.2, min_points=32):
    """prompt_stem.py:211-240 (detached form)."""
    z, target, mask = z.float().flatten(1), target.float().flatten(1), mask.flatten(1)
    w = mask.float()
    s = torch.ones(z.shape[0])
    t = torch.zeros_like(s)
    ok = w.sum(1) >= min_points
    for it in range(iters + 1):
        n = w.sum(1).clamp_min(1)
        sx, sy = (w * z).sum(1), (w * target).sum(1)
        sxx, sxy = (w * z * z).sum(1), (w * z * target).sum(1)
        den = n * sxx - sx * sx
        s_new = torch.where(den > 1e-12, (n * sxy - sx * sy) / den.clamp_min(1e-12), torch.ones_like(s))
        t_new = (sy - s_new * sx) / n
        s, t = torch.where(ok, s_new, s), torch.where(ok, t_new, t)
        if it == iters:
            break
        r = (s[:, None] * z + t[:, None] - target).abs() / target.clamp_min(1e-3)
        r = torch.where(mask, r, torch.full_like(r, float("inf")))
        k = ((1 - trim) * mask.sum(1)).long().clamp_min(min_points)
        thr = torch.stack([ri.kthvalue(min(int(ki), ri.numel())).values for ri, ki in zip(r, k)])
        w = (mask & (r <= thr[:, None])).float()
    return s, t


def _fake_quant(x, scale):
    s = torch.as_tensor(scale, dtype=torch.float32).clamp_min(1e-12)
    return torch.clamp(torch.round(x / s), -QMAX, QMAX) * s


def _weight_fq(w):
    dims = list(range(1, w.ndim))
    return _fake_quant(w, w.abs().amax(dim=dims, keepdim=True) / QMAX)


def column_nmap(z):
    """_core.py:269-295: z [B, H, W] -> (M, 27) int64, -1 where absent."""
    B, H, W = z.shape
    flat = torch.arange(B * H * W).view(B, H, W)
    out = torch.full((B, H, W, 27), -1, dtype=torch.long)
    v = 0
    for di in (-1, 0, 1):
        for dj in (-1, 0, 1):
            zs = torch.full_like(z, -(1 << 40))
            fs = torch.full_like(flat, -1)
            si0, si1, sj0, sj1 = max(0, -di), min(H, H - di), max(0, -dj), min(W, W - dj)
            zs[:, si0:si1, sj0:sj1] = z[:, si0 + di:si1 + di, sj0 + dj:sj1 + dj]
            fs[:, si0:si1, sj0:sj1] = flat[:, si0 + di:si1 + di, sj0 + dj:sj1 + dj]
            for dz in (-1, 0, 1):
                out[..., v] = torch.where(zs == z + dz, fs, -1)
                v += 1
    return out.view(-1, 27)


def submanifold_conv(x, nmap, weight, bias):
    """_core.py:399-441: out = bias, then per tap the valid rows gather, mm with W[:, v, :], index_add_."""
    Co = weight.shape[0]
    w = weight.reshape(Co, 27, -1)
    out = bias.expand(x.shape[0], Co).clone()
    for v in range(27):
        idx = nmap[:, v]
        rows = (idx >= 0).nonzero().squeeze(1)
        if rows.numel() == 0:
            continue
        out.index_add_(0, rows, x.index_select(0, idx[rows]) @ w[:, v, :].t())
    return out


def step(points, lidar, conf, w, iters=10, resolution=256.0):
    """One int8 (QAT fake-quant) refiner step on the CPU; points [B, H, W, 3], lidar / conf [B, H, W] at the point
    map's size. Returns the refined points (numpy)."""
    f32 = lambda a: torch.as_tensor(np.asarray(a, np.float32))
    pts = f32(points).clone()
    lid, cf = f32(lidar), f32(conf)
    B, H, W, _ = pts.shape
    logz = pts[..., 2]
    # prompt: _lidar_in_affine_frame (the LiDAR is already at the point map's size: nearest resize is the identity)
    c = (cf / 2.0).clamp(0, 1)
    valid = torch.isfinite(lid) & (lid > 0)
    z = torch.exp(logz)
    s, t = fit_scale_shift(z.flatten(1), lid.flatten(1), (valid & (c >= 0.999)).flatten(1), iters=iters)
    d_aff = (lid - t.view(-1, 1, 1)) / s.view(-1, 1, 1).clamp_min(1e-6)
    ok = valid & (d_aff > 1e-4)
    log_d_aff = torch.where(ok, torch.log(d_aff.clamp_min(1e-4)), logz)
    gate = c * ok.float()
    prompt = torch.stack([(log_d_aff - logz) * gate, gate], dim=-1).reshape(-1, 2)
    # voxelise + level-0 map
    zq = torch.round(logz * resolution).long()
    zq = zq - zq.flatten(1).amin(1).view(-1, 1, 1)
    nmap = column_nmap(zq)
    x = F.linear(pts.reshape(-1, 3), f32(w.in_w), f32(w.in_b)) + F.linear(prompt, f32(w.pr_w), f32(w.pr_b))
    for b in w.blocks:
        w1, w2 = _weight_fq(f32(b.w1)), _weight_fq(f32(b.w2))
        h = F.silu(F.layer_norm(x, (x.shape[1],), f32(b.gamma), f32(b.beta), eps=1e-6))
        clip1, clip2 = torch.tensor(b.clip1, dtype=torch.float32), torch.tensor(b.clip2, dtype=torch.float32)
        h = F.silu(submanifold_conv(_fake_quant(h, clip1 / QMAX), nmap, w1, f32(b.b1)))
        x = submanifold_conv(_fake_quant(h, clip2 / QMAX), nmap, w2, f32(b.b2)) + x
    out = F.linear(x, f32(w.out_w), f32(w.out_b))
    pts[..., 2] = logz + out.view(B, H, W)
    return pts.numpy()
