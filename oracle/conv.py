"""Submanifold 3x3x3 convolution restated from submanifold_conv (promptmoge/_fallback/flex_gemm/_core.py:399-441).

out[m] = bias + sum_v W[:, v, :] @ x[nmap[m, v]] with W of the module layout (Co, 3, 3, 3, Ci) -> (Co, 27, Ci)
(_core.py:424), taps in ascending order, each tap gathering its valid rows (nonzero) and adding with index_add_.
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, quant_i8, silu_f32


def _w27(w: np.ndarray) -> np.ndarray:
    return w.reshape(w.shape[0], 27, -1)


def conv_acc_int(x: np.ndarray, nmap: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact integer accumulation, int64 result. Each tap's products are formed as a floating-point GEMM, which is
    exact because every partial sum is an integer of magnitude <= Ci * max|x| * max|w| below the format's 2^24 (fp32)
    or 2^53 (fp64) -- the argument of compress/verify_int8.py:94-97. Taps are then summed in int64."""
    M = x.shape[0]
    w = _w27(np.asarray(w))
    acc = np.zeros((M, w.shape[0]), dtype=np.int64)
    bound = float(x.shape[1]) * float(np.abs(x).max(initial=0)) * float(np.abs(w).max(initial=0))
    ft = np.float32 if bound < 2.0 ** 24 else np.float64
    assert bound < 2.0 ** 53
    xf = x.astype(ft)
    for v in range(27):
        idx = nmap[:, v]
        rows = np.nonzero(idx >= 0)[0]
        if rows.size == 0:
            continue
        g = xf[idx[rows]] @ w[:, v, :].T.astype(ft)
        acc[rows] += g.astype(np.int64)  # rows are unique within one tap, as index_add_ assumes nothing else
    return acc


def conv_float(x: np.ndarray, nmap: np.ndarray, w: np.ndarray, bias=None, dtype=np.float32) -> np.ndarray:
    """The _fallback order in `dtype`: out = 0 + bias, then per tap out[rows] += x[src] @ W_v^T."""
    M = x.shape[0]
    w = _w27(np.asarray(w)).astype(dtype)
    out = np.zeros((M, w.shape[0]), dtype=dtype)
    if bias is not None:
        out += np.asarray(bias, dtype=dtype)
    x = x.astype(dtype)
    for v in range(27):
        idx = nmap[:, v]
        rows = np.nonzero(idx >= 0)[0]
        if rows.size == 0:
            continue
        out[rows] += x[idx[rows]] @ w[:, v, :].T
    return out


def dequant(acc: np.ndarray, a_scale, w_scale: np.ndarray, bias=None) -> np.ndarray:
    """y = (float(acc) * a_scale) * w_scale[n] + bias[n], fp32 op by op (SparseConvInt8.metal:107, 139)."""
    y = acc.astype(np.float32) * np.float32(a_scale)
    y = y * w_scale.astype(np.float32)[None, :]
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)[None, :]
    return y


def epilogue_q(acc, a_scale, w_scale, bias, out_mult) -> np.ndarray:
    """conv1 epilogue: bias, SiLU, requantise for the next layer with mult = 127/clip (SparseConvInt8.metal:101-111)."""
    return quant_i8(silu_f32(dequant(acc, a_scale, w_scale, bias)), out_mult)


def epilogue_qlin(acc, a_scale, w_scale, bias, out_mult) -> np.ndarray:
    """Requantisation with no activation, clamp(rint(y * out_mult), +-127) of the dequantised y: with a_scale =
    out_mult = 1 and no bias it is the per-channel q = clamp(rint(acc * m[n]), +-127) of the conv microbenchmark."""
    return quant_i8(dequant(acc, a_scale, w_scale, bias), out_mult)


def epilogue_r(acc, a_scale, w_scale, bias, skip) -> np.ndarray:
    """conv2 epilogue: bias plus the block's identity skip (SparseConvInt8.metal:133-141; flex_sparse_blocks.py:234)."""
    return dequant(acc, a_scale, w_scale, bias) + skip.astype(np.float32)


def dense_correlation(coords: np.ndarray, shape, x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Independent check of the sparse conv: scatter features into a dense grid and cross-correlate with the 3x3x3
    kernel by shifting the whole grid (F.conv3d's convention, _core.py:8-15), then read the active voxels.
    float64; small grids only."""
    B, X, Y, Z = shape
    Ci = x.shape[1]
    w = _w27(np.asarray(w)).astype(np.float64)
    g = np.zeros((B, X + 2, Y + 2, Z + 2, Ci))
    b, i, j, k = coords.T
    g[b, i + 1, j + 1, k + 1] = x
    out = np.zeros((coords.shape[0], w.shape[0]))
    v = 0
    for di in (-1, 0, 1):
        for dj in (-1, 0, 1):
            for dk in (-1, 0, 1):
                nb = g[b, i + 1 + di, j + 1 + dj, k + 1 + dk]
                out += nb @ w[:, v, :].T
                v += 1
    return out
