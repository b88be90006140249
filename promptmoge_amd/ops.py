"""Torch-facing wrappers of the libpmg entry points.

Tensors are device tensors (HIP); every call enqueues on torch's current stream and returns without synchronising.
Inputs are validated here (device, dtype, shape, contiguity) before the C ABI validates them again.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import EPI_ACC, EPI_BIAS, EPI_Q, EPI_QLIN, EPI_R, EPI_RLN, EPI_ROUT, EPI_SILU, ConvEpilogue, call, lib

__all__ = [
    "voxelize", "nmap_column", "nmap_hash", "row_order", "nmap_from_rows", "kmap_compact", "spconv_i8",
    "spconv_i8_ordered", "spconv_f16", "spconv_bf16",
    "spconv_f32", "spconv_col", "ln_silu_quant", "ln_silu_f16", "fit_scale_shift", "fit_prompt", "fit_final",
    "post_depth",
    "math_device", "gauge_poly",
    "nearest_fill",
    "EPI_ACC", "EPI_Q", "EPI_R", "EPI_BIAS", "EPI_SILU", "EPI_RLN", "EPI_ROUT", "EPI_QLIN",
]


def _stream() -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _dev(t: torch.Tensor, name: str, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def math_device(op: int, x: torch.Tensor) -> torch.Tensor:
    """Test hook: op 0/1/2 = exp/log/silu of x; op 3 = the epilogues' int8 SiLU code of x[:, 0] at mult x[:, 1]."""
    x = _dev(x, "x", torch.float32)
    if op == 3:
        if x.ndim != 2 or x.shape[1] != 2:
            raise ValueError("op 3 takes (n, 2) pairs (y, mult)")
        out = torch.empty((x.shape[0],), dtype=torch.float32, device=x.device)
        n = x.shape[0]
    else:
        out = torch.empty_like(x)
        n = x.numel()
    call("pmg_math_device", op, _p(x), _p(out), n, _stream())
    return out


# ------------------------------------------------------------------------------------------------------------- (1)
def voxelize(logz: torch.Tensor, resolution: float = 256.0, stride: int = 1,
             shape: Optional[Tuple[int, int, int]] = None):
    """zq = rint(logz * resolution) and per-batch (min, max). logz: [B, H, W] (stride 1) or the point map
    [B, H, W, 3] viewed from its third channel (pass points[..., 2:] with stride 3 and shape=(B, H, W))."""
    if shape is None:
        B, H, W = logz.shape
    else:
        B, H, W = shape
    dev = logz.device
    zq = torch.empty((B, H, W), dtype=torch.int32, device=dev)
    zmin = torch.empty((B,), dtype=torch.int32, device=dev)
    zmax = torch.empty((B,), dtype=torch.int32, device=dev)
    call("pmg_voxelize", _p(logz), stride, B, H, W, float(resolution), _p(zq), _p(zmin), _p(zmax), _stream())
    return zq, zmin, zmax


# ------------------------------------------------------------------------------------------------------------- (2)
def nmap_column(zq: torch.Tensor, zmin: Optional[torch.Tensor] = None, *, taps: bool = True, rows: bool = False,
                coords: bool = False):
    """Level-0 column-stencil map. Returns (nmap_t [27, M] | None, tile_mask [ceil(M/16)], nmap_rows [M, 27] | None,
    coords [M, 4] | None)."""
    zq = _dev(zq, "zq", torch.int32)
    B, H, W = zq.shape
    M = B * H * W
    dev = zq.device
    nt = torch.empty((27, M), dtype=torch.int32, device=dev) if taps else None
    nr = torch.empty((M, 27), dtype=torch.int32, device=dev) if rows else None
    tm = torch.empty(((M + 15) // 16,), dtype=torch.int32, device=dev)
    cd = torch.empty((M, 4), dtype=torch.int32, device=dev) if coords else None
    if coords and zmin is None:
        raise ValueError("coords need zmin")
    call("pmg_nmap_column", _p(zq), _p(zmin), B, H, W, _p(nt), _p(nr), _p(tm), _p(cd), _stream())
    return nt, tm, nr, cd


def nmap_hash(coords: torch.Tensor, sparse_shape: Sequence[int], *, taps: bool = True, rows: bool = False,
              row_mask: bool = False):
    """Generic map over unique (b, x, y, z) coords. Returns (nmap_t [27, M] | None, tile_mask, nmap_rows | None), and
    with row_mask=True a fourth item, each row's 27-bit tap mask [M] (int32)."""
    coords = _dev(coords, "coords", torch.int32)
    if coords.ndim != 2 or coords.shape[1] != 4:
        raise ValueError("coords must be (M, 4)")
    M = coords.shape[0]
    dev = coords.device
    nt = torch.empty((27, M), dtype=torch.int32, device=dev) if taps else None
    nr = torch.empty((M, 27), dtype=torch.int32, device=dev) if rows else None
    tm = torch.empty(((M + 15) // 16,), dtype=torch.int32, device=dev)
    ws_bytes = lib().pmg_hash_workspace_bytes(M)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    rm = torch.empty((M,), dtype=torch.int32, device=dev) if row_mask else None
    shape = (C.c_int64 * 4)(*[int(s) for s in sparse_shape[:4]])
    call("pmg_nmap_hash", _p(coords), M, shape, _p(nt), _p(nr), _p(tm), _p(rm), _p(ws), ws_bytes, _stream())
    return (nt, tm, nr, rm) if row_mask else (nt, tm, nr)


def sorted_workspace(sparse_shape: Sequence[int], device) -> torch.Tensor:
    """A workspace for nmap_sorted: its status word zeroed, the rest uninitialised (reusable by later calls)."""
    shape = (C.c_int64 * 4)(*[int(s) for s in sparse_shape[:4]])
    nbytes = lib().pmg_sorted_workspace_bytes(shape)
    if nbytes == 0:
        raise ValueError("nmap_sorted: more than 2^31 (b, x, y) columns")
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=device)
    ws[:256].zero_()
    return ws


def sorted_workspace_fits(sparse_shape: Sequence[int]) -> bool:
    """Whether nmap_sorted takes this sparse shape (at most 2^31 (b, x, y) columns)."""
    shape = (C.c_int64 * 4)(*[int(s) for s in sparse_shape[:4]])
    return lib().pmg_sorted_workspace_bytes(shape) > 0


def sorted_status(ws: torch.Tensor) -> int:
    """The status word of an nmap_sorted workspace (reads it back): 0 while every call saw sorted coordinates."""
    return int(ws[:4].view(torch.int32).item())


def nmap_sorted(coords: torch.Tensor, sparse_shape: Sequence[int], *, taps: bool = True, rows: bool = False,
                row_mask: bool = False, workspace: Optional[torch.Tensor] = None):
    """nmap_hash for coords in strictly increasing _linearise order (the order _SortedIndex sorts into): the same
    outputs, from the (b, x, y) columns' row runs. The order is checked on the device; `workspace` (sorted_workspace)
    carries the sticky status word, read with sorted_status -- without one, a fresh workspace is checked here (one
    synchronisation) and a violation raises."""
    coords = _dev(coords, "coords", torch.int32)
    if coords.ndim != 2 or coords.shape[1] != 4:
        raise ValueError("coords must be (M, 4)")
    M = coords.shape[0]
    dev = coords.device
    own = workspace is None
    ws = sorted_workspace(sparse_shape, dev) if own else workspace
    nt = torch.empty((27, M), dtype=torch.int32, device=dev) if taps else None
    nr = torch.empty((M, 27), dtype=torch.int32, device=dev) if rows else None
    tm = torch.empty(((M + 15) // 16,), dtype=torch.int32, device=dev)
    rm = torch.empty((M,), dtype=torch.int32, device=dev) if row_mask else None
    shape = (C.c_int64 * 4)(*[int(s) for s in sparse_shape[:4]])
    call("pmg_nmap_sorted", _p(coords), M, shape, _p(nt), _p(nr), _p(tm), _p(rm), _p(ws), ws.numel(), _stream())
    if own and sorted_status(ws) != 0:
        raise ValueError("nmap_sorted: coords are not in increasing _linearise order (or lie outside sparse_shape)")
    return (nt, tm, nr, rm) if row_mask else (nt, tm, nr)


ROW_ORDER_WINDOW = 1 << 18


def row_order(row_mask: torch.Tensor, nmap_rows: Optional[torch.Tensor] = None, window: int = ROW_ORDER_WINDOW):
    """Processing order for spconv_i8_ordered: within windows of `window` consecutive rows (0: one window), rows
    stably sorted by their 27-bit tap mask; the tile masks [ceil(M/16)] of that order and, given the row-major map
    (nmap_hash(rows=True)), the tap-major map in that order (the map spconv_i8_ordered reads).
    Returns (order [M] int32, order_tile_mask, nmap_o [27, M] | None)."""
    row_mask = _dev(row_mask, "row_mask", torch.int32)
    M = row_mask.shape[0]
    dev = row_mask.device
    order = torch.empty((M,), dtype=torch.int32, device=dev)
    otm = torch.empty(((M + 15) // 16,), dtype=torch.int32, device=dev)
    nmo = None
    if nmap_rows is not None:
        nmap_rows = _dev(nmap_rows, "nmap_rows", torch.int32)
        if tuple(nmap_rows.shape) != (M, 27) or not nmap_rows.is_contiguous():
            raise ValueError("nmap_rows must be a contiguous (M, 27) map")
        nmo = torch.empty((27, M), dtype=torch.int32, device=dev)
    ws_bytes = lib().pmg_row_order_workspace_bytes(M)
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    call("pmg_row_order", _p(row_mask), _p(nmap_rows), M, int(window), _p(order), _p(otm), _p(nmo), _p(ws), ws_bytes, _stream())
    return order, otm, nmo


def pool_cache(coords: torch.Tensor, sparse_shape: Sequence[int], stride: Sequence[int],
               out_sparse_shape: Sequence[int]):
    """build_pool_cache (_core.py:339-395), perfect partition, output coordinates not given. Returns
    (out_coords [N, 4] int32, parent [M] int32, seg_indices [M] int32, seg_offsets [N + 1] int64). Reads the
    output count back to the host once (the reference's int(...) sync)."""
    coords = _dev(coords, "coords", torch.int32)
    if coords.ndim != 2 or coords.shape[1] != 4:
        raise ValueError("coords must be (M, 4)")
    M = coords.shape[0]
    dev = coords.device
    oc = torch.empty((max(M, 1), 4), dtype=torch.int32, device=dev)
    parent = torch.empty((M,), dtype=torch.int32, device=dev)
    seg = torch.empty((M,), dtype=torch.int32, device=dev)
    offs = torch.empty((M + 1,), dtype=torch.int64, device=dev)
    counts = torch.empty((2,), dtype=torch.int64, device=dev)
    ws_bytes = lib().pmg_pool_cache_workspace_bytes(M)
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    shp = (C.c_int64 * 4)(*[int(v) for v in sparse_shape[:4]])
    st = (C.c_int32 * 3)(*[int(v) for v in stride[:3]])
    osh = (C.c_int64 * 4)(*[int(v) for v in out_sparse_shape[:4]])
    call("pmg_pool_cache", _p(coords), M, shp, st, osh, _p(oc), _p(parent), _p(seg), _p(offs), _p(counts), _p(ws),
         ws_bytes, _stream())
    n, bad = (int(v) for v in counts.cpu())
    if bad:
        raise ValueError(f"pool_cache: {bad} voxels lie outside the sparse shape {tuple(sparse_shape[:4])}")
    return oc[:n], parent, seg, offs[:n + 1]


def sparse_pool(feats: torch.Tensor, seg_indices: torch.Tensor, seg_offsets: torch.Tensor, num_out: int,
                reduce: str = "mean") -> torch.Tensor:
    """sparse_pool's reduction (_core.py:464-476) over a pool cache: fp32 sums in input order, / group size."""
    if reduce not in ("mean", "sum"):
        raise NotImplementedError(f"reduce={reduce!r} not needed by MoGe")
    feats = _dev(feats, "feats", torch.float32)
    M, Cc = feats.shape
    out = torch.empty((num_out, Cc), dtype=torch.float32, device=feats.device)
    call("pmg_sparse_pool", _p(feats), M, Cc, _p(seg_indices), _p(seg_offsets), num_out, 1 if reduce == "mean" else 0,
         _p(out), _stream())
    return out


def sparse_upsample(feats: torch.Tensor, parent: torch.Tensor) -> torch.Tensor:
    """Nearest upsampling (_core.py:484-505): out[i] = feats[parent[i]]."""
    feats = _dev(feats, "feats")
    parent = _dev(parent, "parent", torch.int32)
    out = torch.empty((parent.shape[0],) + tuple(feats.shape[1:]), dtype=feats.dtype, device=feats.device)
    row_bytes = feats[0].numel() * feats.element_size() if feats.shape[0] else 16
    call("pmg_sparse_upsample", _p(feats), row_bytes, _p(parent), parent.shape[0], _p(out), _stream())
    return out


def nmap_from_rows(nmap_rows: torch.Tensor):
    """(M, 27) map -> (nmap_t [27, M], tile_mask)."""
    nmap_rows = _dev(nmap_rows, "nmap_rows", torch.int32)
    M = nmap_rows.shape[0]
    nt = torch.empty((27, M), dtype=torch.int32, device=nmap_rows.device)
    tm = torch.empty(((M + 15) // 16,), dtype=torch.int32, device=nmap_rows.device)
    call("pmg_nmap_from_rows", _p(nmap_rows), M, _p(nt), _p(tm), _stream())
    return nt, tm


def kmap_compact(nmap_t: torch.Tensor, capacity: Optional[int] = None):
    """Per-tap compacted kernel maps: (offsets [28] int64, out_rows, in_rows). Synchronises the stream."""
    nmap_t = _dev(nmap_t, "nmap_t", torch.int32)
    M = nmap_t.shape[1]
    cap = 27 * M if capacity is None else int(capacity)
    dev = nmap_t.device
    off = torch.empty((28,), dtype=torch.int64, device=dev)
    out_rows = torch.empty((max(cap, 1),), dtype=torch.int32, device=dev)
    in_rows = torch.empty((max(cap, 1),), dtype=torch.int32, device=dev)
    ws_bytes = lib().pmg_kmap_workspace_bytes(M)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    call("pmg_kmap_compact", _p(nmap_t), M, _p(off), _p(out_rows), _p(in_rows), cap, _p(ws), ws_bytes, _stream())
    total = int(off[27].item())
    return off, out_rows[:total], in_rows[:total]


# ------------------------------------------------------------------------------------------------------------- (3)
def _conv_out(M: int, Co: int, epilogue: int, elt: str, dev) -> torch.Tensor:
    if elt == "i8":
        dt = {EPI_ACC: torch.int32, EPI_Q: torch.int8, EPI_QLIN: torch.int8}.get(epilogue, torch.float32)
    elif elt == "f16":
        dt = torch.float16 if epilogue == EPI_SILU else torch.float32
    else:
        dt = torch.float32
    return torch.empty((M, Co), dtype=dt, device=dev)


def spconv_i8(x: torch.Tensor, nmap_t: torch.Tensor, tile_mask: torch.Tensor, w: torch.Tensor, epilogue: int = EPI_ACC,
              *, a_scale: float = 1.0, w_scale: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
              out_mult: float = 1.0, skip: Optional[torch.Tensor] = None,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """int8 submanifold conv. x: (M, Ci) int8; w: (Co, 3, 3, 3, Ci) or (Co, 27, Ci) int8."""
    x = _dev(x, "x", torch.int8)
    w = _dev(w, "w", torch.int8)
    M, Ci = x.shape
    Co = w.shape[0]
    if w.numel() != Co * 27 * Ci:
        raise ValueError("weight must be (Co, 3, 3, 3, Ci)")
    if out is None:
        out = _conv_out(M, Co, epilogue, "i8", x.device)
    call("pmg_spconv_i8", _p(x), _p(nmap_t), _p(tile_mask), M, Ci, Co, _p(w), epilogue, float(a_scale), _p(w_scale),
         _p(bias), float(out_mult), _p(skip), _p(out), _stream())
    return out


def spconv_i8_ordered(x: torch.Tensor, nmap_o: torch.Tensor, order: torch.Tensor, order_tile_mask: torch.Tensor,
                      w: torch.Tensor, epilogue: int = EPI_ACC, *, a_scale: float = 1.0,
                      w_scale: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                      out_mult: float = 1.0, skip: Optional[torch.Tensor] = None,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """spconv_i8 with rows processed in `order`, reading the map permuted into that order (row_order's nmap_o):
    identical results, fewer taps per chunk of rows. Ci = Co = 64, 128."""
    x = _dev(x, "x", torch.int8)
    w = _dev(w, "w", torch.int8)
    order = _dev(order, "order", torch.int32)
    M, Ci = x.shape
    Co = w.shape[0]
    if w.numel() != Co * 27 * Ci:
        raise ValueError("weight must be (Co, 3, 3, 3, Ci)")
    if out is None:
        out = _conv_out(M, Co, epilogue, "i8", x.device)
    call("pmg_spconv_i8_ordered", _p(x), _p(nmap_o), _p(order), _p(order_tile_mask), M, Ci, Co, _p(w), epilogue,
         float(a_scale), _p(w_scale), _p(bias), float(out_mult), _p(skip), _p(out), _stream())
    return out


def spconv_f16(x: torch.Tensor, nmap_t: torch.Tensor, tile_mask: torch.Tensor, w: torch.Tensor,
               epilogue: int = EPI_ACC, *, bias: Optional[torch.Tensor] = None, skip: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    x = _dev(x, "x", torch.float16)
    w = _dev(w, "w", torch.float16)
    M, Ci = x.shape
    Co = w.shape[0]
    if w.numel() != Co * 27 * Ci:
        raise ValueError("weight must be (Co, 3, 3, 3, Ci)")
    if out is None:
        out = _conv_out(M, Co, epilogue, "f16", x.device)
    call("pmg_spconv_f16", _p(x), _p(nmap_t), _p(tile_mask), M, Ci, Co, _p(w), epilogue, _p(bias), _p(skip), _p(out),
         _stream())
    return out


def spconv_bf16(x: torch.Tensor, nmap_t: torch.Tensor, tile_mask: torch.Tensor, w: torch.Tensor,
                epilogue: int = EPI_ACC, *, bias: Optional[torch.Tensor] = None, skip: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16 features (M, Ci) and weights (Co, 3, 3, 3, Ci): bf16 MFMA, fp32 accumulation, fp32 output (M, Co);
    epilogues ACC, BIAS (+ bias) and R (+ bias + skip)."""
    x = _dev(x, "x", torch.bfloat16)
    w = _dev(w, "w", torch.bfloat16)
    M, Ci = x.shape
    Co = w.shape[0]
    if w.numel() != Co * 27 * Ci:
        raise ValueError("weight must be (Co, 3, 3, 3, Ci)")
    if out is None:
        out = torch.empty((M, Co), dtype=torch.float32, device=x.device)
    call("pmg_spconv_bf16", _p(x), _p(nmap_t), _p(tile_mask), M, Ci, Co, _p(w), epilogue, _p(bias), _p(skip), _p(out),
         _stream())
    return out


def spconv_f32(x: torch.Tensor, nmap_t: torch.Tensor, tile_mask: torch.Tensor, w: torch.Tensor,
               bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    x = _dev(x, "x", torch.float32)
    w = _dev(w, "w", torch.float32)
    M, Ci = x.shape
    Co = w.shape[0]
    if w.numel() != Co * 27 * Ci:
        raise ValueError("weight must be (Co, 3, 3, 3, Ci)")
    out = torch.empty((M, Co), dtype=torch.float32, device=x.device)
    call("pmg_spconv_f32", _p(x), _p(nmap_t), _p(tile_mask), M, Ci, Co, _p(w),
         EPI_BIAS if bias is not None else EPI_ACC, _p(bias), _p(out), _stream())
    return out


def spconv_col(x: torch.Tensor, zq: torch.Tensor, w: torch.Tensor, epilogue: int = EPI_ACC, *, a_scale: float = 1.0,
               w_scale: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None, out_mult: float = 1.0,
               skip: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
               ln_gamma: Optional[torch.Tensor] = None, ln_beta: Optional[torch.Tensor] = None, ln_eps: float = 1e-6,
               next_mult: float = 1.0, next_q: Optional[torch.Tensor] = None, out_w: Optional[torch.Tensor] = None,
               out_b: Optional[torch.Tensor] = None, points: Optional[torch.Tensor] = None,
               points_out: Optional[torch.Tensor] = None):
    """Level-0 conv from the voxel keys zq [B, H, W] (no neighbour map). x: (M, C) int8 or fp16; w: (C, 3, 3, 3, C).
    Returns the main output (or points_out for EPI_ROUT)."""
    prec = {torch.int8: _lib.PREC_INT8, torch.float16: _lib.PREC_FP16}[x.dtype]
    x = _dev(x, "x")
    zq = _dev(zq, "zq", torch.int32)
    w = _dev(w, "w", x.dtype)
    B, H, W = zq.shape
    M, Cc = x.shape
    if M != B * H * W or w.numel() != Cc * 27 * Cc:
        raise ValueError("shape mismatch")
    if out is None and epilogue != EPI_ROUT:
        if epilogue == EPI_ACC:
            dt = torch.int32 if prec == _lib.PREC_INT8 else torch.float32
        elif epilogue == EPI_Q:
            dt = x.dtype
        else:
            dt = torch.float32
        out = torch.empty((M, Cc), dtype=dt, device=x.device)
    e = ConvEpilogue(float(a_scale), _p(w_scale), _p(bias), float(out_mult), _p(skip), _p(out), _p(ln_gamma),
                     _p(ln_beta), float(ln_eps), float(next_mult), _p(next_q), _p(out_w), _p(out_b), _p(points),
                     _p(points_out))
    call("pmg_spconv_col", prec, _p(x), _p(zq), B, H, W, Cc, _p(w), epilogue, C.byref(e), _stream())
    return points_out if epilogue == EPI_ROUT else out


def ln_silu_quant(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, out_mult: float,
                  eps: float = 1e-6) -> torch.Tensor:
    x = _dev(x, "x", torch.float32)
    M, Cc = x.shape
    q = torch.empty((M, Cc), dtype=torch.int8, device=x.device)
    call("pmg_ln_silu_quant", _p(x), M, Cc, _p(gamma), _p(beta), float(eps), float(out_mult), _p(q), _stream())
    return q


def ln_silu_f16(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    x = _dev(x, "x", torch.float32)
    M, Cc = x.shape
    h = torch.empty((M, Cc), dtype=torch.float16, device=x.device)
    call("pmg_ln_silu_f16", _p(x), M, Cc, _p(gamma), _p(beta), float(eps), _p(h), _stream())
    return h


# ------------------------------------------------------------------------------------------------------------- (4)
_FIT_WS: dict = {}


def _fit_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """The metric fit's workspace: zero-filled once, then reused by every call on the same (device, stream), since the
    fit kernel leaves it ready for the next launch. Calls on one stream are ordered, so they never share it at once."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _FIT_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros((nbytes,), dtype=torch.uint8, device=device)
        _FIT_WS[key] = ws
    return ws


def fit_scale_shift(z: torch.Tensor, target: torch.Tensor, mask: torch.Tensor, iters: int = 4, trim: float = 0.2,
                    min_points: int = 32, differentiable: bool = False, *, return_info: bool = False):
    """fit_scale_shift (prompt_stem.py:211-240) on the GPU, same arguments: z, target, mask [B, ...] (flattened
    from dim 1). Returns s, t: [B] fp32 (and, with return_info, info [B, 5] int32 = count, k, ok, threshold bits,
    error flag). A batch item whose device-wide wait expired (the grid could not run co-resident) gets s = t = NaN
    and error flag 1; the workspace is ready for the next call either way. The result carries no gradient;
    `differentiable=True` under grad mode is refused."""
    if differentiable and torch.is_grad_enabled() and z.requires_grad:
        raise NotImplementedError("the GPU metric fit is inference-only (differentiable=True needs autograd)")
    z = _dev(z.float().reshape(z.shape[0], -1).contiguous(), "z")
    target = _dev(target.float().reshape(target.shape[0], -1).contiguous(), "target")
    m8 = _dev(mask.reshape(mask.shape[0], -1).to(torch.uint8).contiguous(), "mask")
    B, N = z.shape
    st = torch.empty((B, 2), dtype=torch.float32, device=z.device)
    info = torch.empty((B, 5), dtype=torch.int32, device=z.device)
    ws_bytes = lib().pmg_fit_workspace_bytes(N, iters)
    ws = _fit_workspace(ws_bytes, z.device)
    call("pmg_fit_scale_shift", _p(z), _p(target), _p(m8), B, N, int(iters), float(trim), int(min_points), _p(st),
         _p(info), _p(ws), ws_bytes, _stream())
    if return_info:
        return st[:, 0], st[:, 1], info
    return st[:, 0], st[:, 1]


def fit_prompt(points: torch.Tensor, lidar: torch.Tensor, conf: torch.Tensor, iters: int = 4, trim: float = 0.2,
               min_points: int = 32, return_info: bool = False):
    """Prompt fit of _lidar_in_affine_frame (v3.py:362-378) on the point map [B, H, W, 3] and LiDAR [B, dh, dw]."""
    points = _dev(points, "points", torch.float32)
    lidar = _dev(lidar.float().contiguous(), "lidar")
    conf = _dev(conf.float().contiguous(), "conf")
    B, H, W, _ = points.shape
    dh, dw = lidar.shape[-2:]
    st = torch.empty((B, 2), dtype=torch.float32, device=points.device)
    info = torch.empty((B, 5), dtype=torch.int32, device=points.device)
    ws_bytes = lib().pmg_fit_workspace_bytes(H * W, iters)
    ws = _fit_workspace(ws_bytes, points.device)
    call("pmg_fit_prompt", points.data_ptr() + 8, 3, _p(lidar), _p(conf), B, H, W, dh, dw, int(iters), float(trim),
         int(min_points), _p(st), _p(info), _p(ws), ws_bytes, _stream())
    if return_info:
        return st[:, 0], st[:, 1], info
    return st[:, 0], st[:, 1]


def fit_final(points: torch.Tensor, lidar: torch.Tensor, conf: torch.Tensor, mask_binary: Optional[torch.Tensor] = None,
              iters: int = 4, trim: float = 0.2, min_points: int = 32, return_info: bool = False):
    """Final metric fit (v3.py:768-778) of the depth exp(logz) of the point map [B, H, W, 3] against LiDAR
    [B, dh, dw] at LiDAR resolution (area-pooled depth). Returns (s, t) [B] (and the per-item info [B, 5])."""
    points = _dev(points, "points", torch.float32)
    lidar = _dev(lidar.float().contiguous(), "lidar")
    conf = _dev(conf.float().contiguous(), "conf")
    B, H, W, _ = points.shape
    dh, dw = lidar.shape[-2:]
    mb = None
    if mask_binary is not None:
        mb = _dev(mask_binary.to(torch.uint8).contiguous(), "mask_binary")
        if mb.numel() != B * H * W:
            raise ValueError("mask_binary must be [B, H, W]")
    st = torch.empty((B, 2), dtype=torch.float32, device=points.device)
    info = torch.empty((B, 5), dtype=torch.int32, device=points.device)
    ws_bytes = lib().pmg_fit_final_workspace_bytes(B, dh, dw, iters)
    ws = _fit_workspace(ws_bytes, points.device)
    call("pmg_fit_final", points.data_ptr() + 8, 3, _p(lidar), _p(conf), _p(mb), B, H, W, dh, dw, int(iters),
         float(trim), int(min_points), _p(st), _p(info), _p(ws), ws_bytes, _stream())
    if return_info:
        return st[:, 0], st[:, 1], info
    return st[:, 0], st[:, 1]

def post_depth(points: torch.Tensor, st: torch.Tensor, mask: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """post_depth (MetricFit.metal:200-211; v3.py:776): metric depth s * exp(logz) + t of the point map
    [B, H, W, 3] with the per-frame final fit st [B, 2] (read on the device, no synchronisation); +inf where mask
    [B, H, W] (bool / uint8, optional) is false or the depth is not positive. Returns [B, H, W] fp32."""
    points = _dev(points, "points", torch.float32)
    st = _dev(st.float().contiguous(), "st")
    B, H, W, _ = points.shape
    if st.shape != (B, 2):
        raise ValueError("st must be [B, 2]")
    m8 = None
    if mask is not None:
        m8 = _dev(mask.to(torch.uint8).contiguous(), "mask")
        if m8.numel() != B * H * W:
            raise ValueError("mask must be [B, H, W]")
    if out is None:
        out = torch.empty((B, H, W), dtype=torch.float32, device=points.device)
    call("pmg_post_depth", points.data_ptr() + 8, 3, _p(m8), B, H, W, _p(st), _p(out), _stream())
    return out


def nearest_fill(depth: torch.Tensor, conf: Optional[torch.Tensor] = None, *, return_index: bool = False,
                 out: Optional[Tuple[torch.Tensor, Optional[torch.Tensor]]] = None):
    """nearest_fill (promptmoge/model.py:61-72) on the GPU for depth (and conf) maps [..., h, w] fp32.

    Pixels with depth <= 0 (or NaN) take the depth of the nearest valid pixel -- the pixel scipy's exact EDT
    feature transform names: least distance, ties to the smaller column, then the smaller row -- and conf 1; an
    image without a valid pixel is returned as it is. Returns (depth, conf | None[, src_index]); `out` may be the
    inputs themselves (in-place fill). src_index holds i*w + j of each pixel's source (-1: no valid pixel).
    """
    depth = _dev(depth, "depth", torch.float32)
    if depth.ndim < 2:
        raise ValueError("depth must be [..., h, w]")
    h, w = depth.shape[-2:]
    B = depth.numel() // max(h * w, 1)
    if conf is not None:
        conf = _dev(conf, "conf", torch.float32)
        if conf.shape != depth.shape:
            raise ValueError("conf must have the shape of depth")
    if out is None:
        d_out = torch.empty_like(depth)
        c_out = torch.empty_like(conf) if conf is not None else None
    else:
        d_out, c_out = out
        d_out = _dev(d_out, "depth_out", torch.float32)
        if d_out.shape != depth.shape or (conf is not None and (c_out is None or c_out.shape != conf.shape)):
            raise ValueError("out must match the inputs")
    idx = torch.empty(depth.shape, dtype=torch.int32, device=depth.device) if return_index else None
    if depth.numel() > 0:
        ws_bytes = lib().pmg_nearest_fill_workspace_bytes(B, h, w)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=depth.device)
        call("pmg_nearest_fill", _p(depth), _p(conf), B, h, w, _p(d_out), _p(c_out) if conf is not None else None,
             _p(idx), _p(ws), ws_bytes, _stream())
    if return_index:
        return d_out, c_out, idx
    return d_out, c_out


def gauge_poly(depth: torch.Tensor, lidar: torch.Tensor, conf: Optional[torch.Tensor] = None, degree: int = 2,
               iters: int = 3, *, return_coef: bool = False):
    """MoGeModel.prompt_gauge_poly (moge/model/v3.py:151-183) on the GPU: the [B, H, W] correction exp(poly(u, v))
    fitted by IRLS to log(prompt / area-pooled prediction) on confident prompt pixels (fewer than 200: 1).

    depth [B, H, W] fp32; lidar (and conf, or None) [B, h, w] or [B, 1, h, w] fp32. With return_coef also the
    per-frame coefficients [B, 8] (basis order (1, u, v, u^2, uv, v^2); [:, 7] is 1 where the frame was fitted).
    """
    depth = _dev(depth, "depth", torch.float32)
    if depth.ndim != 3:
        raise ValueError("depth must be [B, H, W]")
    B, H, W = depth.shape
    lidar = _dev(lidar, "lidar", torch.float32)
    h, w = lidar.shape[-2:]
    if lidar.numel() != B * h * w:
        raise ValueError("lidar must be [B, h, w] or [B, 1, h, w]")
    if conf is not None:
        conf = _dev(conf, "conf", torch.float32)
        if conf.numel() != B * h * w:
            raise ValueError("conf must match lidar")
    corr = torch.empty_like(depth)
    coef = torch.empty((B, 8), dtype=torch.float32, device=depth.device)
    ws_bytes = lib().pmg_gauge_poly_workspace_bytes(B, h, w)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=depth.device)
    call("pmg_gauge_poly", _p(depth), B, H, W, _p(lidar), _p(conf), h, w, int(degree), int(iters), _p(corr),
         _p(coef), _p(ws), ws_bytes, _stream())
    return (corr, coef) if return_coef else corr
