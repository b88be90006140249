"""Seeded synthetic inputs and refiner weights for the benchmark configurations.

Nothing here is a checkpoint or a dataset: scenes are ray-cast piecewise-planar rooms, and refiner weights are drawn
from fixed distributions with the int8 quantisation of the reference's QAT contract (moge/model/modules/qat.py).

Configurations (the workloads of the benchmark; M = voxels at level 0 = H*W, one voxel per pixel as in
MoGeModel._voxelize, moge/model/v3.py:305-344):
  B  240x320, fx=fy=260, cx=160, cy=120; int8, 4 conv layers (2 residual blocks), C=32, fit iters 10, K=1
  A  480x640, fx=fy=520, cx=320, cy=240; int8, 6 conv layers (3 blocks), C=48, fit iters 10, K=1  (headline)
  T  480x640 as A; fp16 teacher, 6 conv layers, C=64, K=3
  H  756x1008, fx=fy=819, cx=504, cy=378; planes + 1-3 cm cylinders; 20 % LiDAR holes nearest-filled; int8,
     6 layers, C=64, K=3
  U  1,000,000 unique voxels in a 1024^3 grid from random planes and sphere shells (9.9 active taps per voxel);
     C in {64, 128} (conv microbench)
"""
from __future__ import annotations

import dataclasses
from typing import Dict, List, Optional

import numpy as np


@dataclasses.dataclass(frozen=True)
class StepConfig:
    name: str
    H: int
    W: int
    fx: float
    fy: float
    cx: float
    cy: float
    C: int
    n_blocks: int
    precision: str  # "int8" | "fp16"
    fit_iters: int = 10
    steps: int = 1
    cylinders: bool = False
    holes: float = 0.0
    seed: int = 0

    @property
    def M(self) -> int:
        return self.H * self.W


CONFIGS: Dict[str, StepConfig] = {
    "B": StepConfig("B", 240, 320, 260.0, 260.0, 160.0, 120.0, 32, 2, "int8", seed=11),
    "A": StepConfig("A", 480, 640, 520.0, 520.0, 320.0, 240.0, 48, 3, "int8", seed=12),
    "T": StepConfig("T", 480, 640, 520.0, 520.0, 320.0, 240.0, 64, 3, "fp16", steps=3, seed=13),
    "H": StepConfig("H", 756, 1008, 819.0, 819.0, 504.0, 378.0, 64, 3, "int8", steps=3, cylinders=True, holes=0.2,
                    seed=14),
}

# The affine frame of the synthetic network prediction: lidar ~= S0 * exp(logz) + T0.
S0, T0 = 1.3, 0.05


@dataclasses.dataclass
class Scene:
    points: np.ndarray  # [H, W, 3] fp32 (x/z, y/z, logz) in the network's affine frame
    lidar: np.ndarray   # [H, W] fp32 metres (0 = missing)
    conf: np.ndarray    # [H, W] fp32 in {0, 1, 2}
    depth: np.ndarray   # [H, W] fp64 ground truth


def _planes(rng, H, W, fx, fy, cx, cy, dx, dy) -> np.ndarray:
    D = np.full((H, W), np.inf)
    n_planes = int(rng.integers(6, 11))
    for _ in range(n_planes):
        while True:
            u, v = rng.uniform(0, W), rng.uniform(0, H)
            p = rng.uniform(0.8, 6.0) * np.array([(u - cx) / fx, (v - cy) / fy, 1.0])
            n = rng.normal(size=3)
            n /= np.linalg.norm(n)
            if n @ p > 0:
                n = -n
            if -(n @ p) / np.linalg.norm(p) > 0.25:
                break
        c = n @ p
        nd = n[0] * dx[None, :] + n[1] * dy[:, None] + n[2]
        with np.errstate(divide="ignore", invalid="ignore"):
            t = np.where(nd < -1e-6, c / nd, np.inf)
        D = np.minimum(D, np.where(t > 0, t, np.inf))
    return D


def _cylinders(rng, D, dx, dy) -> np.ndarray:
    """Thin vertical and horizontal cylinders (radius 1-3 cm) in front of the planes."""
    for _ in range(int(rng.integers(8, 16))):
        rho = rng.uniform(0.01, 0.03)
        z0 = rng.uniform(0.8, 4.0)
        if rng.random() < 0.5:  # vertical: axis along y through (x0, z0)
            x0 = rng.uniform(-0.6, 0.6) * z0
            a = dx * dx + 1.0
            b = -2.0 * (dx * x0 + z0)
            c = x0 * x0 + z0 * z0 - rho * rho
            disc = b * b - 4 * a * c
            t = np.where(disc >= 0, (-b - np.sqrt(np.maximum(disc, 0))) / (2 * a), np.inf)
            D = np.minimum(D, np.where(t > 0, t, np.inf)[None, :])
        else:  # horizontal: axis along x through (y0, z0)
            y0 = rng.uniform(-0.45, 0.45) * z0
            a = dy * dy + 1.0
            b = -2.0 * (dy * y0 + z0)
            c = y0 * y0 + z0 * z0 - rho * rho
            disc = b * b - 4 * a * c
            t = np.where(disc >= 0, (-b - np.sqrt(np.maximum(disc, 0))) / (2 * a), np.inf)
            D = np.minimum(D, np.where(t > 0, t, np.inf)[:, None])
    return D


def nearest_fill(depth: np.ndarray, conf: np.ndarray):
    """promptmoge.model.nearest_fill (promptmoge/model.py:61-72): missing pixels take the nearest valid value and
    confidence 1. Host-side (SciPy exact EDT), as in the reference."""
    valid = depth > 0
    if valid.all() or not valid.any():
        return depth, conf
    from scipy import ndimage

    idx = ndimage.distance_transform_edt(~valid, return_distances=False, return_indices=True)
    return depth[tuple(idx)], np.where(valid, conf, 1).astype(conf.dtype)


def make_scene(cfg: StepConfig, seed: Optional[int] = None, fill: bool = True) -> Scene:
    """Ray-cast piecewise-planar room (6-10 planes, depth clipped to [0.5, 6] m) plus sigma = 5 mm Gaussian noise:
    that depth map is the LiDAR prompt (same resolution, 3 % gross outliers, i.i.d. confidence in {0, 1, 2} with
    P = (0.1, 0.2, 0.7)) and, mapped into an affine frame (depth ~= 1.3 * exp(logz) + 0.05), the network's point
    map (x/z, y/z, logz) that the refiner voxelises. With holes (config H) the LiDAR is nearest-filled here unless
    fill=False, which returns it with the holes at 0 (for a device-side fill)."""
    rng = np.random.default_rng(cfg.seed if seed is None else seed)
    H, W = cfg.H, cfg.W
    dx = (np.arange(W) - cfg.cx) / cfg.fx
    dy = (np.arange(H) - cfg.cy) / cfg.fy
    D = _planes(rng, H, W, cfg.fx, cfg.fy, cfg.cx, cfg.cy, dx, dy)
    if cfg.cylinders:
        D = _cylinders(rng, D, dx, dy)
    D = np.where(np.isfinite(D), D, 6.0)
    D = np.clip(D, 0.5, 6.0)
    D_obs = D + rng.normal(0.0, 0.005, size=D.shape)
    out = rng.random(D.shape) < 0.03
    lidar = np.where(out, D_obs * rng.uniform(0.5, 1.5, size=D.shape), D_obs)
    conf = rng.choice(np.array([0.0, 1.0, 2.0]), size=D.shape, p=[0.1, 0.2, 0.7])
    if cfg.holes > 0:
        hole = rng.random(D.shape) < cfg.holes
        lidar = np.where(hole, 0.0, lidar)
        if fill:
            lidar, conf = nearest_fill(lidar, conf)
    d_net = (D_obs - T0) / S0
    points = np.stack(
        [np.broadcast_to(dx[None, :], (H, W)), np.broadcast_to(dy[:, None], (H, W)), np.log(d_net)], axis=-1
    ).astype(np.float32)
    return Scene(points=np.ascontiguousarray(points), lidar=lidar.astype(np.float32), conf=conf.astype(np.float32),
                 depth=D)


# ------------------------------------------------------------------------------------------------------------------
# Conv microbench voxel set.
def _sphere_shell(rng, grid) -> np.ndarray:
    """A naive digital sphere: on each of the 6 caps where one axis dominates the normal, one voxel per column of
    that axis (the surface point over the column's centre), so a voxel has ~9 of its 27 neighbour positions
    occupied, as on a flat patch."""
    c = rng.uniform(0.2 * grid, 0.8 * grid, size=3)
    r = rng.uniform(20, 110)
    out = []
    for ax in range(3):
        oth = [a for a in range(3) if a != ax]
        a = np.arange(int(c[oth[0]] - r) - 1, int(c[oth[0]] + r) + 2) + 0.5
        b = np.arange(int(c[oth[1]] - r) - 1, int(c[oth[1]] + r) + 2) + 0.5
        A, B = np.meshgrid(a, b, indexing="ij")
        A, B = A.ravel(), B.ravel()
        da, db = A - c[oth[0]], B - c[oth[1]]
        rem = r * r - da * da - db * db
        h = np.sqrt(np.maximum(rem, 0.0))
        for sgn in (1.0, -1.0):
            dz = sgn * h
            dom = (rem >= 0) & (np.abs(dz) >= np.abs(da)) & (np.abs(dz) >= np.abs(db))
            q = np.zeros((int(dom.sum()), 3), np.int64)
            q[:, oth[0]], q[:, oth[1]] = np.floor(A[dom]), np.floor(B[dom])
            q[:, ax] = np.floor(c[ax] + dz[dom])
            out.append(q)
    return np.concatenate(out)


def make_voxels(n: int = 1_000_000, grid: int = 1024, seed: int = 21) -> np.ndarray:
    """`n` unique voxels (b=0, x, y, z) of a `grid`^3 volume, lexicographically sorted: the union of random plane
    patches, sampled densely (0.35-voxel spacing, so oblique patches are a few voxels thick), and sphere shells drawn
    as naive digital surfaces (_sphere_shell). Occupancy is surface-like: 9.9 of the 27 neighbour positions of a
    voxel are occupied on average at the default size (BASELINE's ~8-12)."""
    rng = np.random.default_rng(seed)
    keys: List[np.ndarray] = []
    seen = np.zeros(0, dtype=np.int64)
    total = 0
    while total < n:
        if rng.random() < 0.5:
            # plane patch: origin + a*u + b*v, sampled at 0.35-voxel spacing
            o = rng.uniform(0.1 * grid, 0.9 * grid, size=3)
            nrm = rng.normal(size=3)
            nrm /= np.linalg.norm(nrm)
            u = np.cross(nrm, rng.normal(size=3))
            u /= np.linalg.norm(u)
            v = np.cross(nrm, u)
            half = rng.uniform(40, 160)
            a = np.arange(-half, half, 0.35)
            A, Bm = np.meshgrid(a, a, indexing="ij")
            q = np.floor(o + A.reshape(-1, 1) * u + Bm.reshape(-1, 1) * v).astype(np.int64)
        else:
            q = _sphere_shell(rng, grid)
        ok = np.all((q >= 0) & (q < grid), axis=1)
        q = q[ok]
        k = (q[:, 0] * grid + q[:, 1]) * grid + q[:, 2]
        k = np.unique(k)
        k = k[~np.isin(k, seen, assume_unique=True)] if seen.size else k
        if total + k.size > n:
            k = k[: n - total]
        keys.append(k)
        seen = np.union1d(seen, k)
        total += k.size
    k = np.sort(np.concatenate(keys))
    coords = np.zeros((k.size, 4), dtype=np.int32)
    coords[:, 1] = k // (grid * grid)
    coords[:, 2] = (k // grid) % grid
    coords[:, 3] = k % grid
    return coords


# ------------------------------------------------------------------------------------------------------------------
# Synthetic refiner weights.
def quantize_weight(w: np.ndarray):
    """Per-output-channel symmetric int8 (WeightFakeQuant, qat.py:52-57 with _fake_quant, qat.py:35-36):
    s = max|W[co]| / 127 (fp32), q = clamp(rint(W / s), -127, 127). Returns (q int8, s fp32 [Co])."""
    w = w.astype(np.float32)
    s = (np.abs(w).reshape(w.shape[0], -1).max(axis=1) / np.float32(127.0)).astype(np.float32)
    s = np.maximum(s, np.float32(1e-12))
    q = np.clip(np.rint(w / s.reshape((-1,) + (1,) * (w.ndim - 1))), -127, 127).astype(np.int8)
    return q, s


def act_scale(clip: float) -> np.float32:
    """Per-tensor activation scale clip / 127 in fp32 (ActFakeQuant.forward, qat.py:98; Refiner.swift:147)."""
    return np.maximum(np.float32(clip) / np.float32(127.0), np.float32(1e-12))


def act_mult(clip: float) -> np.float32:
    """Requantisation multiplier 127 / clip in fp32, as the deployed engine computes it (Refiner.swift:148)."""
    return np.float32(127.0) / np.float32(clip)


@dataclasses.dataclass
class BlockW:
    gamma: np.ndarray
    beta: np.ndarray
    w1: np.ndarray  # (C, 3, 3, 3, C) fp32 master weight
    b1: np.ndarray
    w2: np.ndarray
    b2: np.ndarray
    clip1: float = 1.0  # activation clip of conv1's input
    clip2: float = 1.0  # activation clip of conv2's input


@dataclasses.dataclass
class RefinerW:
    C: int
    in_w: np.ndarray  # (C, 3)
    in_b: np.ndarray
    pr_w: np.ndarray  # (C, 2)
    pr_b: np.ndarray
    out_w: np.ndarray  # (1, C)
    out_b: np.ndarray  # (1,)
    blocks: List[BlockW]



def weights_from_state_dict(sd, stages=("down_stages.0", "bottleneck_stage"), clips=None) -> RefinerW:
    """A single-level refiner's weights from a Sparse3DUNet state dict (sparse_unet.py:176-258), in the names the
    reference's modules give them: input_proj / prompt_proj / out_proj (nn.Linear), and per SparseResBlock3d
    (flex_sparse_blocks.py:50-75) under each stage prefix `<stage>.<k>.`: norm1, conv1, conv2 (weights
    (Co, 3, 3, 3, Ci), nn/__init__.py:30). QAT-wrapped weights are read from `.parametrizations.weight.original`
    (torch.nn.utils.parametrize, qat.py:111); activation clips from the quantisers' `aq_<module_path>.clip`
    buffers (qat.py:76, 112-115), or from `clips` = {module path: clip}; a clip found in neither is NaN, which the
    int8 refiner refuses (naming the layer). Tensors may be torch tensors or arrays."""
    f32 = lambda t: np.asarray(t.detach().cpu().float().numpy() if hasattr(t, "detach") else t, dtype=np.float32)

    def get(name: str):
        if name in sd:
            return f32(sd[name])
        base, _, leaf = name.rpartition(".")
        alt = f"{base}.parametrizations.{leaf}.original"
        if alt in sd:
            return f32(sd[alt])
        raise KeyError(name)

    def clip(path: str) -> float:
        if clips is not None and path in clips:
            return float(clips[path])
        key = "aq_" + path.replace(".", "_") + ".clip"
        if key in sd:
            return float(f32(sd[key]))
        return float("nan")  # unknown: the fp16 / fp32 refiner never reads it, the int8 one refuses it

    in_w, in_b = get("input_proj.weight"), get("input_proj.bias")
    C = in_w.shape[0]
    if "prompt_proj.weight" in sd or "prompt_proj.parametrizations.weight.original" in sd:
        pr_w, pr_b = get("prompt_proj.weight"), get("prompt_proj.bias")
    else:
        pr_w, pr_b = np.zeros((C, 2), np.float32), np.zeros((C,), np.float32)
    blocks = []
    for stage in stages:
        k = 0
        while f"{stage}.{k}.norm1.weight" in sd:
            p = f"{stage}.{k}"
            blocks.append(BlockW(get(f"{p}.norm1.weight"), get(f"{p}.norm1.bias"), get(f"{p}.conv1.weight"),
                                 get(f"{p}.conv1.bias"), get(f"{p}.conv2.weight"), get(f"{p}.conv2.bias"),
                                 clip(f"{p}.conv1"), clip(f"{p}.conv2")))
            k += 1
    if not blocks:
        raise ValueError(f"no SparseResBlock3d found under {stages}")
    return RefinerW(C, in_w, in_b, pr_w, pr_b, get("out_proj.weight").reshape(1, C), get("out_proj.bias"), blocks)

def _f16(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float16).astype(np.float32)


def make_weights(C: int, n_blocks: int, seed: int = 0, precision: str = "int8") -> RefinerW:
    """Single-level refiner: input_proj (3->C) + prompt_proj (2->C), n_blocks SparseResBlock3d(C), out_proj (C->1).
    Conv weights ~ N(0, 0.05); biases, LayerNorm affine ~ N(0, 0.05) (gamma around 1), rounded to fp16 as deployed.
    fp16 teacher weights are rounded to fp16 too. Activation clips are calibrated by `calibrate`."""
    rng = np.random.default_rng(1000 + seed)
    f32 = np.float32
    blocks = []
    for _ in range(n_blocks):
        w1 = rng.normal(0, 0.05, size=(C, 3, 3, 3, C)).astype(f32)
        w2 = rng.normal(0, 0.05, size=(C, 3, 3, 3, C)).astype(f32)
        if precision == "fp16":
            w1, w2 = _f16(w1), _f16(w2)
        blocks.append(BlockW(gamma=_f16(1.0 + rng.normal(0, 0.05, size=C)), beta=_f16(rng.normal(0, 0.05, size=C)),
                             w1=w1, b1=_f16(rng.normal(0, 0.05, size=C)), w2=w2, b2=_f16(rng.normal(0, 0.05, size=C))))
    return RefinerW(
        C=C,
        in_w=rng.normal(0, 0.5, size=(C, 3)).astype(f32), in_b=rng.normal(0, 0.05, size=C).astype(f32),
        pr_w=rng.normal(0, 0.5, size=(C, 2)).astype(f32), pr_b=rng.normal(0, 0.05, size=C).astype(f32),
        out_w=rng.normal(0, 0.05, size=(1, C)).astype(f32), out_b=rng.normal(0, 0.01, size=1).astype(f32),
        blocks=blocks,
    )


def _silu(x):
    return x / (1.0 + np.exp(-x))


def calibrate(w: RefinerW, scene: Scene, crop: int = 96, pct: float = 99.95) -> RefinerW:
    """Freezes each conv input's activation clip at the exact 99.95th percentile of |x| (ActFakeQuant, qat.py:60-98)
    from an fp32 forward of the refiner on a central crop of `scene` (prompt features off). Calibration only: the
    arithmetic that is benchmarked and tested is elsewhere."""
    H, W, _ = scene.points.shape
    Hc, Wc = min(crop, H), min(crop, W)  # the whole map when it is smaller than the crop
    h0, w0 = (H - Hc) // 2, (W - Wc) // 2
    pts = scene.points[h0:h0 + Hc, w0:w0 + Wc].astype(np.float64)
    z = np.rint(pts[..., 2].astype(np.float32) * np.float32(256.0)).astype(np.int64)
    x = pts.reshape(-1, 3) @ w.in_w.T.astype(np.float64) + w.in_b
    # column stencil neighbour lists
    idx = np.arange(Hc * Wc).reshape(Hc, Wc)
    taps = []
    for di in (-1, 0, 1):
        for dj in (-1, 0, 1):
            for dz in (-1, 0, 1):
                src = np.full((Hc, Wc), -1)
                zi = np.full((Hc, Wc), np.iinfo(np.int64).min // 4)
                si0, si1, sj0, sj1 = max(0, -di), min(Hc, Hc - di), max(0, -dj), min(Wc, Wc - dj)
                src[si0:si1, sj0:sj1] = idx[si0 + di:si1 + di, sj0 + dj:sj1 + dj]
                zi[si0:si1, sj0:sj1] = z[si0 + di:si1 + di, sj0 + dj:sj1 + dj]
                taps.append(np.where(zi == z + dz, src, -1).reshape(-1))

    def conv(h, wt, b):
        out = np.zeros((h.shape[0], wt.shape[0])) + b
        wr = wt.reshape(wt.shape[0], 27, -1).astype(np.float64)
        for v, nb in enumerate(taps):
            r = nb >= 0
            out[r] += h[nb[r]] @ wr[:, v, :].T
        return out

    for blk in w.blocks:
        mu = x.mean(1, keepdims=True)
        var = x.var(1, keepdims=True)
        h = _silu((x - mu) / np.sqrt(var + 1e-6) * blk.gamma + blk.beta)
        blk.clip1 = float(np.percentile(np.abs(h), pct))
        h = _silu(conv(h, blk.w1, blk.b1))
        blk.clip2 = float(np.percentile(np.abs(h), pct))
        x = x + conv(h, blk.w2, blk.b2)
    return w


def refiner_for(cfg: StepConfig, scene: Optional[Scene] = None) -> RefinerW:
    scene = scene if scene is not None else make_scene(cfg)
    return calibrate(make_weights(cfg.C, cfg.n_blocks, seed=cfg.seed, precision=cfg.precision), scene)
