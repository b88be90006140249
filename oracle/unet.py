"""The multi-level sparse U-Net refiner, restated from the reference (test infrastructure only).

Sparse3DUNet.forward (moge/model/modules/sparse_unet.py:176-258) with SparseResBlock3d, PoolDown and NearestUp
(moge/model/modules/flex_sparse_blocks.py:50-105) over the _fallback flex_gemm structure (submanifold maps,
perfect-partition pooling, nearest upsampling; promptmoge/_fallback/flex_gemm/_core.py:269-505). One composition in
the four arithmetics of oracle/blocks.py: "fp32" (the reference module), "fakequant" (the module under
enable_refiner_qat, qat.py:118-138), "int8" (the deployed integer arithmetic, in the GPU kernels' fp32 op order;
the device engine's sequence, Refiner.swift:224-292 and Refiner.metal:133-322) and "fp16" (the teacher).

Weights: any object with the attributes of promptmoge_amd.unet.UNetW (duck-typed). Linear layers are objects with
`w` (out, in), `b` (out,) and `clip` (the activation clip of their input; unused in "fp32").
"""
from __future__ import annotations

from typing import List, Optional, Sequence

import numpy as np

from .blocks import input_proj, linear, linear_codes, linear_f16, linear_silu_codes, out_proj, resblock, silu
from .pool import pool_cache, sparse_pool, sparse_upsample
from .structure import nmap_column, nmap_sorted, voxelize


# ------------------------------------------------------------------------------------------------- structure
class Level:
    """One resolution level: coords (M, 4) int32 (b, i, j, z) in the reference's row order, the sparse shape
    (B, H, W, Z), the submanifold map (M, 27), and the pool cache from the previous level (parent, seg)."""

    def __init__(self, coords, shape, nmap, parent=None, seg_indices=None, seg_offsets=None):
        self.coords, self.shape, self.nmap = coords, tuple(int(s) for s in shape), nmap
        self.parent, self.seg_indices, self.seg_offsets = parent, seg_indices, seg_offsets

    @property
    def M(self) -> int:
        return int(self.coords.shape[0])


def ceil_div(a: int, b: int) -> int:
    return -(-int(a) // int(b))


def build_levels(coords0: np.ndarray, shape0: Sequence[int], factors: Sequence[int],
                 zkeys: Optional[np.ndarray] = None) -> List[Level]:
    """The structure Sparse3DUNet.forward builds: level 0 from the given coords (the level-0 map is the column
    stencil of _core.py:269-295 when the voxels are one per pixel in raster order, which zkeys [B, H, W] then
    gives; otherwise the sorted map); each next level by PoolDown's perfect-partition pool with stride = factor on
    the three spatial dims and the ceil-divided shape (flex_sparse_blocks.py:36-40, 85-89; _core.py:339-395), with
    its own sorted submanifold map (_core.py:298-304)."""
    coords0 = np.asarray(coords0, np.int32)
    nmap0 = nmap_column(zkeys) if zkeys is not None else nmap_sorted(coords0, shape0)
    levels = [Level(coords0, shape0, nmap0)]
    for f in factors:
        prev = levels[-1]
        B, H, W, Z = prev.shape
        out_shape = (B, ceil_div(H, f), ceil_div(W, f), ceil_div(Z, f))
        oc, parent, seg, offs = pool_cache(prev.coords, prev.shape, (f, f, f), out_shape)
        levels.append(Level(oc, out_shape, nmap_sorted(oc, out_shape), parent, seg, offs))
    return levels


# ------------------------------------------------------------------------------------------------- layers
def sample_rows(planar: np.ndarray, coords: np.ndarray) -> np.ndarray:
    """_sample_encoder_feature (sparse_unet.py:160-174): planar [B, C, h, w] at (b, i, j) of each voxel -> (M, C)."""
    c = np.asarray(coords, np.int64)
    return np.asarray(planar, np.float32)[c[:, 0], :, c[:, 1], c[:, 2]]


# ------------------------------------------------------------------------------------------------- forward
def forward(feats, levels: List[Level], w, encoder_feature, prompt_feats=None, encoder_bias_map=None,
            mode: str = "int8", trace: Optional[dict] = None, record: Optional[dict] = None,
            acc=np.float64) -> np.ndarray:
    """Sparse3DUNet.forward (sparse_unet.py:176-258) on a built structure. Returns (M0,) (out_channels = 1).

    feats (M0, 3) fp32; encoder_feature [B, C_enc, H/16, W/16]; prompt_feats (M0, 2) or None; encoder_bias_map
    [B, C_L, H/16, W/16] or None. trace (optional dict) receives per-stage results (int8: also block codes);
    record (fp32 / fakequant) the input of every quantised layer under its module path (qat.py:118-138). acc: the
    sums of the fp16 mode's convolutions and linears (fp64 exact; fp32 another order)."""
    L = len(levels)
    assert len(w.down) == L and len(w.pool) == L - 1 and len(w.up) == L - 1 and len(w.dec) == L - 1
    feats = np.asarray(feats, np.float32)
    if mode in ("int8", "fp16"):
        res = gate = None
        if prompt_feats is not None:
            pf = np.asarray(prompt_feats, np.float32)
            res, gate = pf[:, 0], pf[:, 1]
        x = input_proj(feats, w, res, gate)                                     # sparse_unet.py:189-192
    else:
        x = feats @ np.asarray(w.in_w, np.float32).T + np.asarray(w.in_b, np.float32)
        if prompt_feats is not None:
            pf = np.asarray(prompt_feats, np.float32)
            x = x + (pf @ np.asarray(w.pr_w, np.float32).T + np.asarray(w.pr_b, np.float32))
        x = x.astype(np.float32)
    tr = trace if trace is not None else None
    skips = []
    for k in range(L):                                                          # sparse_unet.py:223-231
        bt = [] if tr is not None else None
        for j, blk in enumerate(w.down[k]):
            x = resblock(x, levels[k].nmap, blk, mode, bt, record, f"down_stages.{k}.{j}", acc)
        if tr is not None:
            tr[f"down{k}"] = x
            tr[f"down{k}_blocks"] = bt
        if k < L - 1:
            skips.append(x)
            nxt = levels[k + 1]
            pooled = sparse_pool(x, nxt.parent, nxt.M, "mean")                 # flex_sparse_blocks.py:85-90
            x = linear(pooled, w.pool[k], mode, record, f"downsample_blocks.{k}.linear", acc)
            if tr is not None:
                tr[f"pool{k}"] = x
    top = levels[L - 1]
    enc = linear(sample_rows(encoder_feature, top.coords), w.enc, mode, record, "encoder_fuse", acc)  # :233-234
    if tr is not None:
        tr["enc_lin"] = enc
    if encoder_bias_map is not None:
        enc = (enc + sample_rows(encoder_bias_map, top.coords)).astype(np.float32)  # :235-239
    cat = np.concatenate([x, enc], axis=1)
    if mode == "int8":                                                          # :240
        x = linear_codes(linear_silu_codes(cat, w.fuse0, w.fuse2.clip), w.fuse2)
    elif mode == "fp16":
        x = linear_f16(linear_f16(cat, w.fuse0, silu_out=True, acc=acc), w.fuse2, acc=acc)
    else:
        x = linear(silu(linear(cat, w.fuse0, mode, record, "fuse_proj.0")), w.fuse2, mode, record, "fuse_proj.2")
    if tr is not None:
        tr["enc"] = enc
        tr["fuse"] = x
    bt = [] if tr is not None else None
    for j, blk in enumerate(w.bott):                                            # :244-247
        x = resblock(x, top.nmap, blk, mode, bt, record, f"bottleneck_stage.{j}", acc)
    if tr is not None:
        tr["bott"] = x
        tr["bott_blocks"] = bt
    for i in range(L - 1):                                                      # :249-256
        t = L - 2 - i
        lin = linear(x, w.up[i], mode, record, f"upsample_blocks.{i}.linear", acc)  # flex_sparse_blocks.py:99-105
        x = (sparse_upsample(lin, levels[t + 1].parent) + skips[t]).astype(np.float32)
        if tr is not None:
            tr[f"dec{i}_in"] = x
        bt = [] if tr is not None else None
        for j, blk in enumerate(w.dec[i]):
            x = resblock(x, levels[t].nmap, blk, mode, bt, record, f"up_stages.{i}.{j}", acc)
        if tr is not None:
            tr[f"dec{i}"] = x
            tr[f"dec{i}_blocks"] = bt
    if mode in ("int8", "fp16"):
        return out_proj(x, w)                                                   # :258
    return (x @ np.asarray(w.out_w, np.float32).reshape(1, -1).T).reshape(-1) + np.float32(np.asarray(w.out_b)[0])


def forward_from_points(points, w, encoder_feature, prompt_feats=None, encoder_bias_map=None, mode="int8",
                        resolution=256.0, trace=None):
    """_refine_logz's refiner call (v3.py:346-357) on a point map [B, H, W, 3]: _voxelize (v3.py:305-344), the
    structure, the forward. Returns (out (M0,), levels)."""
    pts = np.asarray(points, np.float32)
    B, H, W, _ = pts.shape
    zq, coords, zext, _ = voxelize(pts, resolution)
    levels = build_levels(coords, (B, H, W, zext), w.factors, zkeys=zq)
    out = forward(pts.reshape(-1, 3), levels, w, encoder_feature, prompt_feats, encoder_bias_map, mode, trace)
    return out, levels


def calibrate(w, levels, feats, encoder_feature, prompt_feats=None, encoder_bias_map=None, pct: float = 99.95):
    """Activation clips for synthetic weights: each quantised layer's clip set to the exact `pct` percentile of |x|
    of its input in one fp32 forward (ActFakeQuant's statistic, qat.py:60-87, without the EMA and subsampling).
    Returns a copy of `w` with the clips set (conv pairs: clip1 / clip2)."""
    import copy

    rec: dict = {}
    forward(feats, levels, w, encoder_feature, prompt_feats, encoder_bias_map, mode="fp32", record=rec)
    out = copy.deepcopy(w)
    pc = lambda x: float(np.percentile(np.abs(x), pct))
    for path, layer in out.quantised_layers().items():
        if hasattr(layer, "clip1"):
            layer.clip1, layer.clip2 = pc(rec[path + ".conv1"]), pc(rec[path + ".conv2"])
        else:
            layer.clip = pc(rec[path])
    return out


# ------------------------------------------------------------------------------------------------- refine step
def step(points, lidar, conf, w, encoder_feature, encoder_bias_map=None, *, iters=10, trim=0.2, min_points=32,
         use_prompt=True, soft_gate=False, final_fit=False, post_depth=False, resolution=256.0,
         output_gate_on=False, gate_floor=0.1, anchor=0.0, st_given=None, st_anchor_given=None,
         trace: Optional[dict] = None):
    """One refine-loop step with the multi-level refiner (v3.py:547-576): prompt fit of _lidar_in_affine_frame
    (v3.py:362-378), the (residual, gate) prompt features (v3.py:548-555), _refine_logz (v3.py:346-360) with this
    Sparse3DUNet, logz + out, the output gate (v3.py:565-569), the elastic anchor (v3.py:570-573), the final metric
    fit at LiDAR resolution (v3.py:768-778) and post_depth (MetricFit.metal:200-211). The int8 arithmetic of
    `forward`; the steps around it are oracle/refiner.py's.

    st_given / st_anchor_given = (s [B], t [B]) replace the prompt / anchor fit's result (that fit is then not run),
    so that a device whose fit was checked against fit_f64 within its tolerance is compared on identical inputs
    after it. Returns (points [B, H, W, 3], prompt (s, t) or None, final (s, t) or None, depth [B, H, W] or None)."""
    from .fit import final_inputs, fit_f64, prompt_inputs
    from .fit import post_depth as post_depth_fn
    from .refiner import anchor_pull, output_gate, prompt_feats

    pts = np.array(points, dtype=np.float32, copy=True)
    B, H, W, _ = pts.shape
    st = None
    pf = None
    if use_prompt:
        z, tg, m, d, c = prompt_inputs(pts, lidar, conf)
        if st_given is None:
            st = fit_f64(z, tg, m, iters, trim, min_points)
        else:
            st = (np.asarray(st_given[0], np.float32).reshape(B), np.asarray(st_given[1], np.float32).reshape(B))
        r, g = prompt_feats(pts, d, c, st[0], st[1], soft_gate)
        pf = np.stack([r.reshape(-1), g.reshape(-1)], 1)
    delta, levels = forward_from_points(pts, w, encoder_feature, pf, encoder_bias_map, "int8", resolution, trace)
    cur = pts[..., 2].copy()
    pts[..., 2] = pts[..., 2] + delta.reshape(B, H, W)
    if output_gate_on or anchor > 0:
        _, _, _, d_, c_ = prompt_inputs(pts, lidar, conf)
    if output_gate_on:
        pts[..., 2] = output_gate(cur, pts[..., 2], d_, c_, gate_floor)
    if trace is not None:
        trace["before_anchor"] = pts.copy()
    if anchor > 0:
        if st_anchor_given is None:
            z, tg, m, _, _ = prompt_inputs(pts, lidar, conf)
            sa = fit_f64(z, tg, m, iters, trim, min_points)
        else:
            sa = (np.asarray(st_anchor_given[0], np.float32).reshape(B),
                  np.asarray(st_anchor_given[1], np.float32).reshape(B))
        pts[..., 2] = anchor_pull(pts[..., 2], d_, c_, sa[0], sa[1], anchor)
    fin = depth = None
    if final_fit:
        z, tg, m = final_inputs(pts, lidar, conf)
        fin = fit_f64(z, tg, m, iters, trim, min_points)
        if post_depth:
            depth = post_depth_fn(pts, fin)
    if trace is not None:
        trace["levels"] = levels
        trace["prompt_feats"] = pf
    return pts, st, fin, depth
