"""fp32 arithmetic restated operation by operation in NumPy float32, matching promptmoge_amd/csrc/pmg_math.h.

NumPy float32 arithmetic is IEEE-754 with every operation individually rounded (no fused multiply-add), which is
exactly how the kernels are compiled (-ffp-contract=off, correctly rounded division and sqrt). Constants are given
by bit pattern so both sides use identical values.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def _f(bits: int) -> np.float32:
    return np.array([bits], dtype=np.uint32).view(np.float32)[0]


LOG2E = _f(0x3FB8AA3B)
LN2_HI = _f(0x3F317200)
LN2_LO = _f(0x35BFBE8E)
I6, I24, I120, I720, I5040 = _f(0x3E2AAAAB), _f(0x3D2AAAAB), _f(0x3C088889), _f(0x3AB60B61), _f(0x39500D01)
C3, C5, C7, C9 = _f(0x3EAAAAAB), _f(0x3E4CCCCD), _f(0x3E124925), _f(0x3DE38E39)
SQRT2 = _f(0x3FB504F3)


_BLOCK = 1 << 16


def _blocked(fn):
    """Evaluates an elementwise function in blocks of 65536 elements (each block's many passes stay in cache); the
    result is the same, element by element."""
    def run(x):
        x = np.asarray(x, dtype=np.float32)
        if x.size <= _BLOCK:
            return fn(x)
        flat = np.ascontiguousarray(x).reshape(-1)
        out = np.empty_like(flat)
        for i in range(0, flat.size, _BLOCK):
            out[i:i + _BLOCK] = fn(flat[i:i + _BLOCK])
        return out.reshape(x.shape)

    run.__doc__ = fn.__doc__
    run.__name__ = fn.__name__
    return run


def rowwise(fn, *arrays, block: int = 8192):
    """fn(*row_blocks) over blocks of `block` rows of arrays sharing their first dimension (None passes through),
    on a few threads, results concatenated: for row-independent fn the result of fn(*arrays), element by element."""
    import concurrent.futures as cf
    import os

    n = next(a.shape[0] for a in arrays if a is not None)
    if n <= block:
        return fn(*arrays)
    starts = list(range(0, n, block))
    part = lambda r0: fn(*[a if a is None else a[r0:r0 + block] for a in arrays])
    with cf.ThreadPoolExecutor(max(1, min(8, os.cpu_count() or 1))) as ex:
        outs = list(ex.map(part, starts))
    return np.concatenate(outs)


@_blocked
def exp_f32(x) -> np.ndarray:
    """Cody-Waite reduction, degree-7 Horner polynomial, exponent-field scaling (pmg_math.h exp_f32)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        kf = np.rint(x * LOG2E)
        r = x - kf * LN2_HI
        r = r - kf * LN2_LO
        p = np.full_like(x, I5040)
        for c in (I720, I120, I24, I6, F32(0.5), F32(1.0), F32(1.0)):
            p = p * r + c
        k = np.clip(np.nan_to_num(kf, nan=0.0), -126, 128).astype(np.int64)
        scale = ((np.minimum(k, 127) + 127).astype(np.uint32) << np.uint32(23)).view(np.float32)
        out = p * scale
        out = np.where(k > 127, (p * _f(254 << 23)) * F32(2.0), out)
        out = np.where(x > F32(88.8), F32(np.inf), out)
        out = np.where(x < F32(-87.0), F32(0.0), out)
        out = np.where(np.isnan(x), x, out)
    return out.astype(np.float32)


@_blocked
def log_f32(x) -> np.ndarray:
    """log(x) = e*ln2 + 2 atanh((m-1)/(m+1)) for positive normal x (pmg_math.h log_f32)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    e = (u >> np.uint32(23)).astype(np.int32) - 127
    m = ((u & np.uint32(0x007FFFFF)) | np.uint32(0x3F800000)).view(np.float32)
    big = m > SQRT2
    m = np.where(big, m * F32(0.5), m)
    e = np.where(big, e + 1, e)
    f = m - F32(1.0)
    s = f / (F32(2.0) + f)
    z = s * s
    R = np.full_like(z, C9)
    R = R * z + C7
    R = R * z + C5
    R = R * z + C3
    R = R * z
    t = s + s * R
    logm = t + t
    ef = e.astype(np.float32)
    return (ef * LN2_HI + (ef * LN2_LO + logm)).astype(np.float32)


def silu_f32(y) -> np.ndarray:
    """y / (1 + exp(-y)) (SparseConvInt8.metal:108)."""
    y = np.asarray(y, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (y / (F32(1.0) + exp_f32(-y))).astype(np.float32)


def quant_f32(y, mult) -> np.ndarray:
    """clamp(rint(y * mult), -127, 127) with mult = 127/clip in fp32: the requantisation of the reference's deployed
    int8 kernels (SparseConvInt8.metal:109, Refiner.metal:120, mult from Refiner.swift:148); round half to even.
    The clamp is max-then-min with "a > b ? a : b" / "a < b ? a : b", as pmg_math.h: a NaN input gives -127."""
    y = np.asarray(y, dtype=np.float32)
    q = np.rint(y * np.asarray(mult, dtype=np.float32))
    q = np.where(q > F32(-127.0), q, F32(-127.0))
    return np.where(q < F32(127.0), q, F32(127.0)).astype(np.float32)


def quant_i8(y, mult) -> np.ndarray:
    return quant_f32(y, mult).astype(np.int8)


def quad_sum(v: np.ndarray) -> np.ndarray:
    """Row sum of (M, C) fp32 in the kernels' fixed order: group g = 0..3 accumulates channels 16j + 4g + i
    (j outer, i inner, from 0), then ((s0 + s1) + (s2 + s3)). C must be a multiple of 16."""
    v = np.asarray(v, dtype=np.float32)
    M, C = v.shape
    vr = v.reshape(M, C // 16, 4, 4)  # [m][j][g][i]
    s = np.zeros((M, 4), dtype=np.float32)
    for j in range(C // 16):
        for i in range(4):
            s = s + vr[:, j, :, i]
    return (s[:, 0] + s[:, 1]) + (s[:, 2] + s[:, 3])


def ln_silu(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Two-pass LayerNorm (quad-order sums), affine, SiLU; fp32 op by op (pmg_rowops.hip ln_silu_row and the
    PMG_EPI_RLN epilogue). The reference's block is `silu(norm1(x))` with nn.LayerNorm(eps=1e-6)
    (flex_sparse_blocks.py:215, 230)."""
    x = np.asarray(x, dtype=np.float32)
    M, C = x.shape
    mean = quad_sum(x) / F32(C)
    d = x - mean[:, None]
    var = quad_sum(d * d) / F32(C)
    rstd = F32(1.0) / np.sqrt(var + F32(eps))
    y = (x - mean[:, None]) * rstd[:, None]
    y = y * gamma.astype(np.float32)
    y = y + beta.astype(np.float32)
    return silu_f32(y)
