"""Voxelisation and neighbour maps, restated from the reference.

Tap order everywhere: v = (di+1)*9 + (dj+1)*3 + (dz+1), the itertools.product order of make_conv_kernel_delta
(promptmoge/_fallback/flex_gemm/_core.py:65-82), centre tap 13.
"""
from __future__ import annotations

import itertools
from typing import Dict, Sequence, Tuple

import numpy as np


def kernel_delta(batch_dims: int = 1) -> np.ndarray:
    """make_conv_kernel_delta((3,3,3), (1,1,1), batch_dims) -- _core.py:65-82."""
    rng = [range(-1, 2)] * 3
    return np.array(list(itertools.product(*[(0,)] * batch_dims, *rng)), dtype=np.int64)


def voxelize(points: np.ndarray, resolution: float = 256.0):
    """MoGeModel._voxelize (moge/model/v3.py:305-344). points [B, H, W, 3] fp32.
    Returns (zq [B, H, W] int64 before the min shift, coords (M, 4) int32, z_extent, zmin [B])."""
    points = np.asarray(points, dtype=np.float32)
    B, H, W, _ = points.shape
    logz = points[..., 2]
    zq = np.rint(logz * np.float32(resolution)).astype(np.int64)          # v3.py:332, torch.round = half to even
    zmin = zq.reshape(B, -1).min(axis=1)                                   # v3.py:333
    z_idx = zq - zmin[:, None, None]                                       # v3.py:334
    z_extent = int(z_idx.max()) + 1                                        # v3.py:335
    b, i, j = np.meshgrid(np.arange(B), np.arange(H), np.arange(W), indexing="ij")
    coords = np.stack([b, i, j, z_idx], axis=-1).reshape(-1, 4).astype(np.int32)   # v3.py:337-340
    return zq, coords, z_extent, zmin


def linearise(coords: np.ndarray, shape: Sequence[int]) -> np.ndarray:
    """_linearise (_core.py:89-94)."""
    key = np.zeros(coords.shape[0], dtype=np.int64)
    for d, extent in enumerate(shape):
        key = key * int(extent) + coords[:, d].astype(np.int64)
    return key


def in_bounds(coords: np.ndarray, shape: Sequence[int]) -> np.ndarray:
    """_in_bounds (_core.py:97-102)."""
    ok = np.ones(coords.shape[0], dtype=bool)
    for d, extent in enumerate(shape):
        ok &= (coords[:, d] >= 0) & (coords[:, d] < int(extent))
    return ok


def nmap_column(z: np.ndarray) -> np.ndarray:
    """_build_submanifold_nmap_column (_core.py:269-295): z [B, H, W] integer map -> (M, 27) int32."""
    B, H, W = z.shape
    z = z.astype(np.int64)
    flat = np.arange(B * H * W, dtype=np.int64).reshape(B, H, W)
    NEG = np.iinfo(np.int64).min // 4
    nmap = np.full((B, H, W, 27), -1, dtype=np.int32)
    for v, (_, di, dj, dz) in enumerate(kernel_delta()):
        zs = np.full_like(z, NEG)
        fs = np.full_like(flat, -1)
        si0, si1 = max(0, -di), min(H, H - di)
        ti0, ti1 = max(0, di), min(H, H + di)
        sj0, sj1 = max(0, -dj), min(W, W - dj)
        tj0, tj1 = max(0, dj), min(W, W + dj)
        if si1 > si0 and sj1 > sj0:
            zs[:, si0:si1, sj0:sj1] = z[:, ti0:ti1, tj0:tj1]
            fs[:, si0:si1, sj0:sj1] = flat[:, ti0:ti1, tj0:tj1]
        nmap[..., v] = np.where(zs == z + dz, fs, -1)
    return nmap.reshape(B * H * W, 27)


def nmap_sorted(coords: np.ndarray, shape: Sequence[int]) -> np.ndarray:
    """_SortedIndex + _build_submanifold_nmap_sorted (_core.py:105-124, 298-304): (M, 4) coords -> (M, 27)."""
    coords = coords.astype(np.int64)
    keys = linearise(coords, shape)
    order = np.argsort(keys, kind="stable")
    sk = keys[order]
    n = keys.shape[0]
    out = np.empty((n, 27), dtype=np.int32)
    for v, d in enumerate(kernel_delta()):
        q = coords + d[None, :]
        ok = in_bounds(q, shape)
        qk = np.where(ok, linearise(q, shape), -1)
        pos = np.searchsorted(sk, qk)
        pc = np.minimum(pos, n - 1)
        hit = ok & (pos < n) & (sk[pc] == qk)
        out[:, v] = np.where(hit, order[pc], -1)
    return out


def nmap_bruteforce(coords: np.ndarray, shape: Sequence[int]) -> np.ndarray:
    """Dictionary of coordinates, 27 lookups per voxel (pure Python; small inputs only)."""
    table: Dict[Tuple[int, ...], int] = {}
    for m, c in enumerate(coords.tolist()):
        table.setdefault(tuple(c), m)
    deltas = kernel_delta().tolist()
    out = np.full((len(coords), 27), -1, dtype=np.int32)
    for m, c in enumerate(coords.tolist()):
        for v, d in enumerate(deltas):
            q = tuple(a + b for a, b in zip(c, d))
            if all(0 <= q[k] < shape[k] for k in range(4)) and q in table:
                out[m, v] = table[q]
    return out


def tile_masks(nmap: np.ndarray, tile: int = 16) -> np.ndarray:
    """Bit v of tile t is set iff any of rows [16t, 16t+16) has a neighbour at tap v."""
    M = nmap.shape[0]
    bits = (nmap >= 0).astype(np.uint64) << np.arange(27, dtype=np.uint64)[None, :]
    rows = np.bitwise_or.reduce(bits, axis=1)
    nt = (M + tile - 1) // tile
    pad = np.zeros(nt * tile, dtype=np.uint64)
    pad[:M] = rows
    return np.bitwise_or.reduce(pad.reshape(nt, tile), axis=1).astype(np.uint32)


def kmap_compact(nmap: np.ndarray):
    """Per-tap compacted kernel maps: rows = nonzero(nmap[:, v] >= 0), src = nmap[rows, v] (_core.py:430-437).
    Returns (offsets [28] int64, out_rows, in_rows)."""
    outs, ins, off = [], [], [0]
    for v in range(27):
        rows = np.nonzero(nmap[:, v] >= 0)[0]
        outs.append(rows.astype(np.int32))
        ins.append(nmap[rows, v].astype(np.int32))
        off.append(off[-1] + rows.size)
    return np.array(off, dtype=np.int64), np.concatenate(outs), np.concatenate(ins)
