"""One refinement step of a single-level refiner, restated from the reference.

Step order (moge/model/v3.py:547-576 with _lidar_in_affine_frame 362-383 and _refine_logz 346-360):
  1. prompt fit:   (s, t) = fit_scale_shift(exp(logz), nearest LiDAR, valid & conf/2 >= 0.999)
  2. prompt feats: d_aff = (d - t) / max(s, 1e-6); ok = valid & d_aff > 1e-4; log_d_aff = ok ? log(max(d_aff, 1e-4))
                   : logz; gate = c*ok (soft: (0.15 + 0.85c)*ok); residual = (log_d_aff - logz) * gate
  3. voxelise + level-0 neighbour map
  4. Sparse3DUNet, single level (sparse_unet.py:189-192, 258): h = input_proj(feats) + prompt_proj(residual, gate);
     SparseResBlock3d x n (flex_sparse_blocks.py:229-234); out_proj
  5. logz += out; with the output gate (v3.py:565-569) logz = cur + g * ((cur + out) - cur), g = floor + (1 - floor)
     * u, u = _lidar_uncertainty (v3.py:386-393); with the elastic anchor beta > 0 (v3.py:570-573) the prompt fit
     is repeated on the refined depth and logz += beta * gate * (log_d_aff - logz) (hard gate)
  6. optionally the same fit on the refined depth

`step` computes the blocks in the deployed integer arithmetic (the QAT contract qat.py:1-16 as executed by
SparseConvInt8.metal / Refiner.metal: int8 activations and weights, exact int32 accumulation, fp32 epilogues,
requantisation by 127/clip) or in fp16 (teacher); every fp32 operation in the order of the GPU kernels. `step_fakequant` is the reference's own
fp32 formulation of the int8 model: _fallback's fp32 conv on fake-quantised operands (qat.py:28-57, 89-106).
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from .blocks import (act_mult, act_scale, fake_quant, input_proj, layer_norm, out_proj, quantize_weight,
                     resblock, silu)
from .conv import conv_float
from .fit import final_inputs, fit_f64, prompt_inputs
from .numerics import F32, ln_silu, log_f32, rowwise
from .structure import nmap_column, voxelize


def prompt_feats(points, d, c, s, t, soft_gate=False):
    """v3.py:379-383 and 552-555, op by op in fp32; d, c [B, H, W] (already nearest-resized)."""
    logz = points[..., 2]
    s = np.asarray(s, dtype=np.float32)[:, None, None]
    t = np.asarray(t, dtype=np.float32)[:, None, None]
    valid = np.isfinite(d) & (d > 0)
    with np.errstate(invalid="ignore", over="ignore"):
        daff = (d - t) / np.maximum(s, F32(1e-6))
    ok = valid & (daff > F32(1e-4))
    lda = np.where(ok, log_f32(np.maximum(np.where(ok, daff, F32(1.0)), F32(1e-4))), logz)
    okf = ok.astype(np.float32)
    gate = (F32(0.15) + F32(0.85) * c) * okf if soft_gate else c * okf
    res = (lda - logz) * gate
    return res.astype(np.float32), gate.astype(np.float32)


def blocks_int8(x, nmap, w, trace=None):
    """The residual blocks in the deployed int8 arithmetic (blocks.resblock); trace receives each block's q1, acc1,
    q2, acc2 and output x."""
    for blk in w.blocks:
        x = resblock(x, nmap, blk, "int8", trace)
    return x


def blocks_fp16(x, nmap, w, trace=None):
    """Teacher: fp16 conv operands, fp32 accumulation (here fp64, then rounded), fp32 residual stream."""
    from .numerics import silu_f32

    for blk in w.blocks:
        h1 = rowwise(lambda xb: ln_silu(xb, blk.gamma, blk.beta).astype(np.float16), x)
        y1 = conv_float(h1.astype(np.float64), nmap, np.asarray(blk.w1, np.float16).astype(np.float64),
                        dtype=np.float64).astype(np.float32)
        h2 = rowwise(lambda yb: silu_f32(yb + np.asarray(blk.b1, np.float32)).astype(np.float16), y1)
        y2 = conv_float(h2.astype(np.float64), nmap, np.asarray(blk.w2, np.float16).astype(np.float64),
                        dtype=np.float64).astype(np.float32)
        x = (y2 + np.asarray(blk.b2, np.float32)) + x
        if trace is not None:
            trace.append(dict(h1=h1, h2=h2, x=x))
    return x


def lidar_uncertainty(d, c):
    """_lidar_uncertainty (v3.py:386-393) on nearest-resized d, c [B, H, W]: 1 - c * (1 - range_uncertainty(d)),
    range_uncertainty = clamp((d - 3) / (5 - 3), 0, 1) (prompt_stem.py:28-29, 41-42); 1 where d is not a value."""
    valid = np.isfinite(d) & (d > 0)
    with np.errstate(invalid="ignore"):
        ru = np.clip((np.where(valid, d, F32(0.0)) - F32(3.0)) / F32(2.0), F32(0.0), F32(1.0))
    u = F32(1.0) - c * (F32(1.0) - ru)
    return np.where(valid, u, F32(1.0)).astype(np.float32)


def output_gate(cur, refined, d, c, floor=0.1):
    """v3.py:567-569: cur + g * (refined - cur), g = floor + (1.0 - floor) * u; the two Python-float constants are
    rounded to fp32 by the tensor arithmetic."""
    g = F32(floor) + F32(1.0 - floor) * lidar_uncertainty(d, c)
    return (cur + g * (refined - cur)).astype(np.float32)


def anchor_pull(logz, d, c, s, t, beta):
    """v3.py:570-573 with _lidar_in_affine_frame's hard gate: logz + beta * gate * (log_d_aff - logz)."""
    s_ = np.asarray(s, dtype=np.float32)[:, None, None]
    t_ = np.asarray(t, dtype=np.float32)[:, None, None]
    valid = np.isfinite(d) & (d > 0)
    with np.errstate(invalid="ignore", over="ignore"):
        daff = (d - t_) / np.maximum(s_, F32(1e-6))
    ok = valid & (daff > F32(1e-4))
    lda = np.where(ok, log_f32(np.maximum(np.where(ok, daff, F32(1.0)), F32(1e-4))), logz)
    gate = c * ok.astype(np.float32)
    return (logz + (F32(beta) * gate) * (lda - logz)).astype(np.float32)


def step(points, lidar, conf, w, *, precision="int8", iters=10, trim=0.2, min_points=32, use_prompt=True,
         soft_gate=False, final_fit=False, resolution=256.0, output_gate_on=False, gate_floor=0.1, anchor=0.0,
         trace: Optional[dict] = None, st_given=None):
    """Returns (refined points [B, H, W, 3], (s, t) prompt fit, (s, t) final fit or None).

    st_given = (s [B], t [B]) replaces the prompt fit's result (the fit is then not run): a test that has checked a
    device's fit against fit_f64 within its tolerance passes the device's (s, t) here, so that everything after the
    fit is compared on identical inputs, bit for bit."""
    pts = np.array(points, dtype=np.float32, copy=True)
    B, H, W, _ = pts.shape
    M = B * H * W
    st = None
    res = gate = None
    if use_prompt:
        z, tg, m, d, c = prompt_inputs(pts, lidar, conf)
        if st_given is None:
            st = fit_f64(z, tg, m, iters, trim, min_points)
        else:
            st = (np.asarray(st_given[0], np.float32).reshape(B), np.asarray(st_given[1], np.float32).reshape(B))
        r, g = prompt_feats(pts, d, c, st[0], st[1], soft_gate)
        res, gate = r.reshape(-1), g.reshape(-1)
    zq, coords, _, _ = voxelize(pts, resolution)
    nmap = nmap_column(zq)
    x = input_proj(pts.reshape(M, 3), w, res, gate)
    blk_trace = [] if trace is not None else None
    x = (blocks_int8 if precision == "int8" else blocks_fp16)(x, nmap, w, blk_trace)
    delta = out_proj(x, w)
    cur = pts[..., 2].copy()
    pts[..., 2] = pts[..., 2] + delta.reshape(B, H, W)
    if output_gate_on or anchor > 0:
        _, _, _, d_, c_ = prompt_inputs(pts, lidar, conf)
    if output_gate_on:
        pts[..., 2] = output_gate(cur, pts[..., 2], d_, c_, gate_floor)
    if anchor > 0:
        z, tg, m, _, _ = prompt_inputs(pts, lidar, conf)
        sa = fit_f64(z, tg, m, iters, trim, min_points)
        pts[..., 2] = anchor_pull(pts[..., 2], d_, c_, sa[0], sa[1], anchor)
    fin = None
    if final_fit:  # v3.py:768-778, at LiDAR resolution
        z, tg, m = final_inputs(pts, lidar, conf)
        fin = fit_f64(z, tg, m, iters, trim, min_points)
    if trace is not None:
        trace.update(zq=zq, nmap=nmap, coords=coords, blocks=blk_trace, x=x, res=res, gate=gate)
    return pts, st, fin


# ------------------------------------------------------------------------------------------------------------------
def blocks_fakequant(x, nmap, w):
    """The reference's fp32 formulation: _fallback conv on fake-quantised operands (qat.py:101-111, 52-57)."""
    for blk in w.blocks:
        x = resblock(x, nmap, blk, "fakequant")
    return x


def step_fakequant(points, lidar, conf, w, *, iters=10, trim=0.2, min_points=32, use_prompt=True, soft_gate=False,
                   resolution=256.0):
    """The int8 step as the reference evaluates it on the CPU (fp32 fake quantisation, torch-style LN and exp)."""
    pts = np.array(points, dtype=np.float32, copy=True)
    B, H, W, _ = pts.shape
    M = B * H * W
    res = gate = None
    if use_prompt:
        z, tg, m, d, c = prompt_inputs(pts, lidar, conf)
        z = np.exp(pts[..., 2]).reshape(B, -1).astype(np.float32)
        s, t = fit_f64(z, tg, m, iters, trim, min_points)
        r, g = prompt_feats(pts, d, c, s, t, soft_gate)
        res, gate = r.reshape(-1), g.reshape(-1)
    zq, _, _, _ = voxelize(pts, resolution)
    nmap = nmap_column(zq)
    x = input_proj(pts.reshape(M, 3), w, res, gate)
    x = blocks_fakequant(x, nmap, w)
    x2 = x @ np.asarray(w.out_w, np.float32).reshape(-1) + np.float32(w.out_b[0])
    pts[..., 2] = pts[..., 2] + x2.reshape(B, H, W).astype(np.float32)
    return pts


def forward(feats, zkeys, H, W, w, prompt_feats=None, precision="int8"):
    """The single-level refiner module (sparse_unet.py:176-258 with one level; blocks flex_sparse_blocks.py:50-75):
    out_proj(blocks(input_proj(feats) (+ prompt_proj(prompt_feats)))) -> (M,) on level-0 voxels keyed by zkeys
    [B, H, W] (raster order; any per-batch offset of the keys gives the same map)."""
    feats = np.asarray(feats, np.float32)
    nmap = nmap_column(np.asarray(zkeys))
    res = gate = None
    if prompt_feats is not None:
        pf = np.asarray(prompt_feats, np.float32)
        res, gate = pf[:, 0], pf[:, 1]
    x = input_proj(feats, w, res, gate)
    x = (blocks_int8 if precision == "int8" else blocks_fp16)(x, nmap, w)
    return out_proj(x, w)
