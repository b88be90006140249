"""Submanifold 3x3x3 convolution restated from submanifold_conv (promptmoge/_fallback/flex_gemm/_core.py:399-441).

out[m] = bias + sum_v W[:, v, :] @ x[nmap[m, v]] with W of the module layout (Co, 3, 3, 3, Ci) -> (Co, 27, Ci)
(_core.py:424), taps in ascending order, each tap gathering its valid rows (nonzero) and adding with index_add_.
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, quant_i8, silu_f32


def _w27(w: np.ndarray) -> np.ndarray:
    return w.reshape(w.shape[0], 27, -1)


def _im2col(x_pad: np.ndarray, nmap: np.ndarray, r0: int, r1: int) -> np.ndarray:
    """Rows r0..r1 of the gathered operand: row m holds the 27 neighbour rows of m, tap-major (zeros where the
    map has -1, which points at the zero row appended to x_pad)."""
    idx = nmap[r0:r1]
    idx = np.where(idx >= 0, idx, x_pad.shape[0] - 1)
    return x_pad[idx].reshape(r1 - r0, -1)


def _tap_shift(nmap: np.ndarray, v: int):
    """(valid rows mask, d) if every neighbour of tap v is row m + d (a level-0 column-stencil map), else None."""
    col = nmap[:, v]
    ok = col >= 0
    if not ok.any():
        return ok, 0
    rows = np.nonzero(ok)[0]
    d = int(col[rows[0]]) - int(rows[0])
    if np.array_equal(col[rows], rows + d):
        return ok, d
    return None


def _shift_taps(nmap: np.ndarray, dtype):
    """Per tap (row mask as 0/1 of `dtype`, d) when the whole map is a column-stencil map (every tap a constant row
    offset), else None."""
    taps = []
    for v in range(27):
        t = _tap_shift(nmap, v)
        if t is None:
            return None
        taps.append((t[0].astype(dtype)[:, None], t[1]))
    return taps


def _im2col_shift(x: np.ndarray, taps, r0: int, r1: int, out: np.ndarray) -> np.ndarray:
    """_im2col for a column-stencil map: tap v's block of rows r0..r1 is the slice x[r0 + d_v : r1 + d_v] times the
    tap's row mask (rows without that neighbour become zero)."""
    M, C = x.shape
    X = out[: r1 - r0]
    for v, (okf, d) in enumerate(taps):
        blk = X[:, v * C:(v + 1) * C]
        lo, hi = max(r0, -d), min(r1, M - d)
        if hi <= lo:
            blk[:] = 0
            continue
        np.multiply(x[lo + d:hi + d], okf[lo:hi], out=blk[lo - r0:hi - r0])
        blk[:lo - r0] = 0
        blk[hi - r0:] = 0
    return X


def _over_chunks(M: int, chunk: int, K: int, dtype, fn) -> None:
    """fn(r0, r1, buf) over the row chunks, on a few threads (each chunk writes only its own rows; numpy's copies
    and GEMMs release the GIL); buf is a per-thread (chunk, K) scratch array."""
    import concurrent.futures as cf
    import os
    import threading

    starts = list(range(0, M, chunk))
    local = threading.local()

    def run(r0):
        if not hasattr(local, "buf"):
            local.buf = np.empty((chunk, K), dtype)
        fn(r0, min(M, r0 + chunk), local.buf)

    workers = max(1, min(8, os.cpu_count() or 1, len(starts)))
    if workers == 1:
        for r0 in starts:
            run(r0)
        return
    with cf.ThreadPoolExecutor(workers) as ex:
        list(ex.map(run, starts))


def conv_acc_int(x: np.ndarray, nmap: np.ndarray, w: np.ndarray, chunk: int = 32768) -> np.ndarray:
    """Exact integer accumulation, int64 result: acc[m, n] = sum_v sum_c W[n, v, c] * x[nmap[m, v], c]. The 27
    taps' gathered rows form one (rows, 27 Ci) operand per chunk of rows, multiplied in fp32 by the (27 Ci, Co)
    weight in K-slices small enough that every partial sum is an integer below 2^24 -- exact in fp32 whatever the
    summation order (the argument of compress/verify_int8.py:94-97) -- and the slices summed in int64."""
    Ci = x.shape[1]
    M = nmap.shape[0]  # output rows: the map's (a map of a subset of rows gathers from all of x)
    w = _w27(np.asarray(w))
    Co = w.shape[0]
    K = 27 * Ci
    bound = float(np.abs(x).max(initial=0)) * float(np.abs(w).max(initial=0))
    step = K if bound == 0 else max(1, min(K, int((2.0 ** 24 - 1) // bound)))
    assert step * bound < 2.0 ** 24
    acc = np.zeros((M, Co), dtype=np.int64)
    wk = np.ascontiguousarray(w.reshape(Co, K).T.astype(np.float32))
    taps = _shift_taps(nmap, np.float32) if M == x.shape[0] else None
    xf = x.astype(np.float32)
    x_pad = None if taps is not None else np.concatenate([xf, np.zeros((1, Ci), np.float32)])

    def rows(r0, r1, buf):
        X = _im2col_shift(xf, taps, r0, r1, buf) if taps is not None else _im2col(x_pad, nmap, r0, r1)
        for k0 in range(0, K, step):
            acc[r0:r1] += (X[:, k0:k0 + step] @ wk[k0:k0 + step]).astype(np.int64)

    _over_chunks(M, 4096 if taps is not None else chunk, K, np.float32, rows)
    return acc


def conv_float(x: np.ndarray, nmap: np.ndarray, w: np.ndarray, bias=None, dtype=np.float32,
               chunk: int = 32768) -> np.ndarray:
    """The _fallback order in fp32: out = 0 + bias, then per tap out[rows] += x[src] @ W_v^T. In float64 (the
    teacher's fp32-accumulation reference, where the order of the fp64 sums is immaterial at its tolerance) as one
    im2col GEMM per chunk of rows. Output rows are the map's."""
    M = nmap.shape[0]
    if dtype == np.float64:
        w = _w27(np.asarray(w)).astype(np.float64)
        Co, Ci = w.shape[0], w.shape[2]
        out = np.zeros((M, Co), dtype=np.float64)
        if bias is not None:
            out += np.asarray(bias, dtype=np.float64)
        wk = np.ascontiguousarray(w.reshape(Co, 27 * Ci).T)
        taps = _shift_taps(nmap, np.float64) if M == x.shape[0] else None
        xf = x.astype(np.float64)
        x_pad = None if taps is not None else np.concatenate([xf, np.zeros((1, Ci))])

        def rows(r0, r1, buf):
            X = _im2col_shift(xf, taps, r0, r1, buf) if taps is not None else _im2col(x_pad, nmap, r0, r1)
            out[r0:r1] += X @ wk

        _over_chunks(M, 4096 if taps is not None else chunk, 27 * Ci, np.float64, rows)
        return out
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
