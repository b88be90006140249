"""The `flex_gemm` operator surface of the reference's fallback (promptmoge/_fallback/flex_gemm/_core.py) on the
MI355X kernels of libpmg.so: neighbour maps from the GPU column stencil or the GPU hash, convolutions on MFMA.

Same names, argument meaning, return values and error style as the reference, so that `promptmoge/model.py:29-30`
selects this package when it is importable as `flex_gemm` (see `promptmoge_amd.flex_gemm.install`). Every
computation runs in libpmg.so; there is no CPU path (the library raises if it is missing). Supported: 3x3x3
kernels, dilation 1, one batch dimension -- what MoGe's refiner uses -- and the perfect-partition pooling and
nearest upsampling of its multi-level U-Net (build_pool_cache with output coordinates given raises
NotImplementedError: MoGe does not use that branch).
"""
from __future__ import annotations

import itertools
from typing import Literal, Optional, Sequence

import torch
from torch import Tensor

from .. import ops as _ops

__all__ = [
    "NeighborCache", "NeighborCacheT", "build_submanifold_cache", "build_pool_cache", "submanifold_conv",
    "sparse_pool", "sparse_upsample", "make_conv_kernel_delta",
]


def _broadcast(arg, D: int, name: str):
    """int -> D-tuple; sequences are checked for length D (nn/__init__.py:_broadcast of the reference)."""
    if arg is None:
        return None
    if isinstance(arg, int):
        return (arg,) * D
    arg = tuple(int(a) for a in arg)
    if len(arg) != D:
        raise AssertionError(f"{name} must have length {D}, got {arg}")
    return arg


def make_conv_kernel_delta(kernel_size: Sequence[int], dilation: Sequence[int], batch_dims: int = 0,
                           dtype: torch.dtype = torch.int32, device: Optional[torch.device] = None) -> Tensor:
    """Offsets of the kernel taps, (V, batch_dims + D), in itertools.product order with the last dimension fastest
    (_core.py:65-82); for 3x3x3 this is tap v = (di+1)*9 + (dj+1)*3 + (dz+1), the order every libpmg map uses."""
    axes = [[0]] * batch_dims + [[o * l for o in range(-(k // 2), k // 2 + 1)] for k, l in zip(kernel_size, dilation)]
    return torch.tensor(list(itertools.product(*axes)), dtype=dtype, device=device)


def _check_supported(kernel_size, dilation, batch_dims: int) -> None:
    if tuple(kernel_size) != (3, 3, 3):
        raise NotImplementedError(f"libpmg submanifold maps support kernel_size (3, 3, 3), got {tuple(kernel_size)}")
    if dilation is not None and tuple(dilation) != (1, 1, 1):
        raise NotImplementedError(f"libpmg submanifold maps support dilation 1, got {tuple(dilation)}")
    if batch_dims != 1:
        raise NotImplementedError("libpmg submanifold maps expect coords (b, x, y, z)")


class NeighborCache:
    """Adjacency of a coord set with itself for the 27-tap submanifold conv (_core.py:131-219).

    `nmap` is the reference's (M, 27) int32 row-major map (-1 = no neighbour), materialised on first access; the
    kernels read the tap-major copy `nmap_t` [27, M] and `tile_mask` (bit v of word t set iff tap v is present in
    rows 16t .. 16t+15), which the GPU map builders write directly."""

    is_transposed = False

    def __init__(self, input_coords: Tensor, output_coords: Tensor, *, nmap: Optional[Tensor] = None,
                 nmap_t: Optional[Tensor] = None, tile_mask: Optional[Tensor] = None,
                 seg_indices: Optional[Tensor] = None, seg_offsets: Optional[Tensor] = None,
                 parent: Optional[Tensor] = None, num_kernels: Optional[int] = None,
                 kernel_size: Optional[tuple] = None, dilation: Optional[tuple] = None, stride: Optional[tuple] = None,
                 input_sparse_shape: Optional[Sequence[int]] = None,
                 output_sparse_shape: Optional[Sequence[int]] = None, symmetric: bool = False,
                 build_backend: str = "hash") -> None:
        self.input_coords = input_coords
        self.output_coords = output_coords
        self._nmap = nmap
        self.nmap_t = nmap_t
        self.tile_mask = tile_mask
        self.seg_indices = seg_indices
        self.seg_offsets = seg_offsets
        self.parent = parent
        self.num_kernels = num_kernels
        self.kernel_size = kernel_size
        self.dilation = dilation
        self.stride = stride
        self.input_sparse_shape = None if input_sparse_shape is None else torch.Size(input_sparse_shape)
        self.output_sparse_shape = None if output_sparse_shape is None else torch.Size(output_sparse_shape)
        self.symmetric = symmetric
        self.build_backend = build_backend
        self._T: Optional[NeighborCacheT] = None

    @property
    def nmap(self) -> Optional[Tensor]:
        if self._nmap is None and self.nmap_t is not None:
            self._nmap = self.nmap_t.t().contiguous()
        return self._nmap

    @property
    def num_input_coords(self) -> int:
        return int(self.input_coords.shape[0])

    @property
    def num_output_coords(self) -> int:
        return int(self.output_coords.shape[0])

    @property
    def T(self) -> "NeighborCacheT":
        if self._T is None:
            self._T = NeighborCacheT(self)
        return self._T

    def transpose(self) -> "NeighborCacheT":
        return self.T

    def assert_match(self, *, input_coords=None, output_coords=None, is_transposed=None, **_kw) -> None:
        """Raises AssertionError for a cache built on other coords (_core.py:197-207)."""
        if input_coords is not None:
            assert input_coords.shape[0] == self.input_coords.shape[0], "stale neighbor cache (input rows)"
            assert input_coords.data_ptr() == self.input_coords.data_ptr() or torch.equal(
                input_coords, self.input_coords), "stale neighbor cache (input coords)"
        if output_coords is not None:
            assert output_coords.shape[0] == self.output_coords.shape[0], "stale neighbor cache (output rows)"
        if is_transposed is not None:
            assert bool(is_transposed) == bool(self.is_transposed)

    def occupancy(self) -> dict:
        """Mean / max / min occupied taps per output row."""
        assert self.nmap_t is not None
        occ = (self.nmap_t >= 0).sum(dim=0).float()
        return {"V": float(self.nmap_t.shape[0]), "mean": float(occ.mean()), "max": float(occ.max()),
                "min": float(occ.min()), "rows": float(self.nmap_t.shape[1])}


class NeighborCacheT:
    """Transposed view of a NeighborCache (_core.py:222-246); only nearest upsampling uses it."""

    is_transposed = True

    def __init__(self, base: NeighborCache) -> None:
        self.base = base
        self.input_coords = base.output_coords
        self.output_coords = base.input_coords
        self.parent = base.parent
        self.input_sparse_shape = base.output_sparse_shape
        self.output_sparse_shape = base.input_sparse_shape
        self.kernel_size = base.kernel_size
        self.stride = base.stride

    @property
    def T(self) -> NeighborCache:
        return self.base

    def assert_match(self, **_kw) -> None:
        return None


def _is_one_voxel_per_column(coords: Tensor, sparse_shape: Sequence[int]) -> bool:
    """True iff coords are exactly (b, i, j, z(b, i, j)) for every pixel, in raster order: MoGe's level 0
    (_voxelize, v3.py:337-340). Compared on the device; one host synchronisation, as in _core.py:249-266."""
    B, H, W = int(sparse_shape[0]), int(sparse_shape[1]), int(sparse_shape[2])
    if coords.ndim != 2 or coords.shape[0] != B * H * W or coords.shape[1] != 4:
        return False
    dev, dt = coords.device, coords.dtype
    eb = torch.arange(B, device=dev, dtype=dt).view(B, 1, 1).expand(B, H, W)
    ei = torch.arange(H, device=dev, dtype=dt).view(1, H, 1).expand(B, H, W)
    ej = torch.arange(W, device=dev, dtype=dt).view(1, 1, W).expand(B, H, W)
    c = coords.view(B, H, W, 4)
    return bool(((c[..., 0] == eb) & (c[..., 1] == ei) & (c[..., 2] == ej)).all().item())


def build_submanifold_cache(coords: Tensor, sparse_shape: Sequence[int], kernel_size: Sequence[int],
                            dilation: Optional[Sequence[int]] = None,
                            backend: Literal["auto", "column", "sorted", "hash"] = "auto") -> NeighborCache:
    """Neighbour map of `coords` with itself (_core.py:307-336). backend "auto" uses the GPU column stencil when the
    coords are one voxel per pixel column in raster order (level 0); otherwise (and for "sorted") the column-run
    map when the coords are in increasing _linearise order (checked on the device, read in one host
    synchronisation, as the column test is), else the GPU hash ("hash": always). All give the reference's sorted
    backend's map."""
    D = len(kernel_size)
    batch_dims = coords.shape[1] - D
    dilation = tuple(dilation) if dilation is not None else (1,) * D
    _check_supported(kernel_size, dilation, batch_dims)
    if not coords.is_cuda:
        raise ValueError("coords must be a GPU tensor")
    c32 = coords.to(torch.int32).contiguous()
    use_column = False
    if backend in ("auto", "column"):
        use_column = _is_one_voxel_per_column(c32, sparse_shape)
        if backend == "column" and not use_column:
            raise ValueError("column backend requested but coords are not one-per-column")
    if use_column:
        B, H, W = int(sparse_shape[0]), int(sparse_shape[1]), int(sparse_shape[2])
        zq = c32[:, 3].contiguous().view(B, H, W)
        nmap_t, tile_mask, _, _ = _ops.nmap_column(zq)
        used = "column"
    else:
        shape4 = [int(s) for s in sparse_shape[:4]]
        used = "hash"
        if backend in ("auto", "sorted") and _ops.sorted_workspace_fits(shape4):
            ws = _ops.sorted_workspace(shape4, c32.device)
            nmap_t, tile_mask, _ = _ops.nmap_sorted(c32, shape4, workspace=ws)
            if _ops.sorted_status(ws) == 0:
                used = "sorted"
        if used == "hash":
            nmap_t, tile_mask, _ = _ops.nmap_hash(c32, shape4)
    return NeighborCache(coords, coords, nmap_t=nmap_t, tile_mask=tile_mask, num_kernels=27,
                         kernel_size=tuple(kernel_size), dilation=dilation, input_sparse_shape=sparse_shape,
                         output_sparse_shape=sparse_shape, symmetric=True, build_backend=used)


def _pad_to(t: Tensor, dim: int, multiple: int) -> Tensor:
    n = t.shape[dim]
    r = (-n) % multiple
    if r == 0:
        return t
    pad = list(t.shape)
    pad[dim] = r
    return torch.cat([t, t.new_zeros(pad)], dim=dim)


def submanifold_conv(feats: Tensor, coords: Tensor, shape: torch.Size, weight: Tensor, bias: Optional[Tensor] = None,
                     *, dilation: Optional[Sequence[int]] = None, neighbor_cache: Optional[NeighborCache] = None,
                     **_ignored):
    """out[m] = bias + sum_v W[:, v, :] @ feats[nmap[m, v]] (the cross-correlation of F.conv3d restricted to the
    active set), weight (Co, 3, 3, 3, Ci) -> (out (M, Co) in feats' dtype, neighbor_cache) (_core.py:399-441).

    fp32 features run the fp32 MFMA kernel (exact fp32 products, fp32 accumulation), fp16 and bf16 the fp16 / bf16
    MFMA kernels with fp32 accumulation (bf16 results rounded back from fp32). Forward only: the kernels have no
    backward."""
    kernel_size = tuple(weight.shape[1:-1])
    D = len(kernel_size)
    sparse_shape = tuple(shape[: coords.shape[1]])
    _check_supported(kernel_size, dilation if dilation is not None else (1,) * D, coords.shape[1] - D)
    if torch.is_grad_enabled() and (feats.requires_grad or weight.requires_grad or
                                    (bias is not None and bias.requires_grad)):
        raise RuntimeError("the libpmg submanifold conv is inference-only; run under torch.no_grad()")
    if neighbor_cache is None:
        neighbor_cache = build_submanifold_cache(coords, sparse_shape, kernel_size, dilation)
    else:
        neighbor_cache.assert_match(input_coords=coords, output_coords=coords, is_transposed=False)
    if neighbor_cache.nmap_t is None:
        neighbor_cache.nmap_t, neighbor_cache.tile_mask = _ops.nmap_from_rows(
            neighbor_cache.nmap.to(torch.int32).contiguous())
    M, Ci = feats.shape
    Co = weight.shape[0]
    if weight.shape[-1] != Ci:
        raise ValueError(f"weight expects {weight.shape[-1]} input channels, feats have {Ci}")
    out_dtype = feats.dtype
    w = weight.detach().reshape(Co, 27, Ci)
    b = None if bias is None else bias.detach().float()
    if feats.dtype == torch.float16:
        x = _pad_to(feats.detach().contiguous(), 1, 8)
        wk = _pad_to(_pad_to(w.to(torch.float16), 2, 8), 0, 16).contiguous()
        bk = None if b is None else _pad_to(b, 0, 16).contiguous()
        out = _ops.spconv_f16(x, neighbor_cache.nmap_t, neighbor_cache.tile_mask, wk,
                              _ops.EPI_BIAS if bk is not None else _ops.EPI_ACC, bias=bk)
    elif feats.dtype == torch.bfloat16:
        x = _pad_to(feats.detach().contiguous(), 1, 8)
        wk = _pad_to(_pad_to(w.to(torch.bfloat16), 2, 8), 0, 16).contiguous()
        bk = None if b is None else _pad_to(b, 0, 16).contiguous()
        out = _ops.spconv_bf16(x, neighbor_cache.nmap_t, neighbor_cache.tile_mask, wk,
                               _ops.EPI_BIAS if bk is not None else _ops.EPI_ACC, bias=bk)
    elif feats.dtype == torch.float32:
        x = _pad_to(feats.detach().float().contiguous(), 1, 4)
        wk = _pad_to(_pad_to(w.float(), 2, 4), 0, 16).contiguous()
        bk = None if b is None else _pad_to(b, 0, 16).contiguous()
        out = _ops.spconv_f32(x, neighbor_cache.nmap_t, neighbor_cache.tile_mask, wk, bias=bk)
    else:
        raise TypeError(f"unsupported feature dtype {feats.dtype}")
    out = out[:, :Co]
    return out.to(out_dtype).contiguous(), neighbor_cache


def build_pool_cache(coords: Tensor, sparse_shape: Sequence[int], kernel_size: Sequence[int], stride: Sequence[int],
                     padding: Sequence[int], output_coords: Optional[Tensor] = None,
                     output_sparse_shape: Optional[Sequence[int]] = None) -> NeighborCache:
    """Perfect-partition pool cache (_core.py:339-395): output coords = the unique floor(coord / stride) in
    increasing _linearise order, `parent` (input row -> output row), `seg_indices` (stable argsort of parent) and
    `seg_offsets`, built on the GPU (pmg_pool_cache). Only kernel == stride and padding == 0, as the reference;
    given output coordinates (the reference's lookup branch, which MoGe does not use) raise NotImplementedError."""
    D = len(kernel_size)
    assert tuple(kernel_size) == tuple(stride), "only kernel == stride supported"
    assert all(p == 0 for p in padding), "only padding == 0 supported"
    batch_dims = coords.shape[1] - D
    if D != 3 or batch_dims != 1:
        raise NotImplementedError("libpmg pooling expects coords (b, x, y, z)")
    if output_sparse_shape is None:
        output_sparse_shape = [int(s) if d < batch_dims else -(-int(s) // int(stride[d - batch_dims]))
                               for d, s in enumerate(sparse_shape)]
    if output_coords is not None:
        raise NotImplementedError("libpmg pooling builds its output coordinates (output_coords must be None)")
    coords_i = coords.to(torch.int32).contiguous()
    out_coords, parent, seg, offs = _ops.pool_cache(coords_i, [int(v) for v in sparse_shape],
                                                    [int(v) for v in stride], [int(v) for v in output_sparse_shape])
    return NeighborCache(coords, out_coords.to(coords.dtype), seg_indices=seg, seg_offsets=offs, parent=parent,
                         kernel_size=tuple(kernel_size), stride=tuple(stride), input_sparse_shape=sparse_shape,
                         output_sparse_shape=output_sparse_shape)


def sparse_pool(feats: Tensor, coords: Tensor, shape: torch.Size, kernel_size, stride=None, padding=None,
                reduce: str = "mean", output_coords: Optional[Tensor] = None, output_shape: Optional[torch.Size] = None,
                neighbor_cache: Optional[NeighborCache] = None):
    """Sparse pooling (_core.py:444-481) -> (feats (N, C), out_coords, out_shape, neighbor_cache). 'mean' and
    'sum'; the rows of each output are summed in input order in fp32 (for fp32 features: the reference's
    index_add_ bit for bit), then divided by the group size for 'mean'."""
    D = len(kernel_size)
    stride = tuple(stride) if stride is not None else tuple(kernel_size)
    padding = tuple(padding) if padding is not None else (0,) * D
    sparse_dim = coords.shape[1]
    sparse_in = tuple(shape[:sparse_dim])
    sparse_out = tuple(output_shape[:sparse_dim]) if output_shape is not None else None
    if reduce not in ("mean", "sum"):
        raise NotImplementedError(f"reduce={reduce!r} not needed by MoGe")
    if neighbor_cache is None:
        neighbor_cache = build_pool_cache(coords, sparse_in, kernel_size, stride, padding, output_coords, sparse_out)
    out_coords = neighbor_cache.output_coords
    num_out = int(out_coords.shape[0])
    C = feats.shape[1]
    x = _pad_to(feats.detach().float().contiguous(), 1, 4)
    acc = _ops.sparse_pool(x, neighbor_cache.seg_indices, neighbor_cache.seg_offsets, num_out, reduce)
    acc = acc[:, :C].to(feats.dtype).contiguous()
    out_shape = torch.Size([*neighbor_cache.output_sparse_shape, C])
    return acc, out_coords, out_shape, neighbor_cache


def sparse_upsample(feats: Tensor, coords: Tensor, shape: torch.Size, scale_factor, *, mode: str = "nearest",
                    output_coords: Optional[Tensor] = None, output_shape: Optional[torch.Size] = None,
                    neighbor_cache=None, **_ignored):
    """Nearest sparse upsampling with the transposed pool cache (_core.py:484-505): out[i] = feats[parent[i]]."""
    assert mode == "nearest", "MoGe only uses nearest upsampling"
    assert neighbor_cache is not None and neighbor_cache.is_transposed, (
        "reference path requires the transposed pool cache (MoGe always supplies it)")
    assert output_coords is not None
    parent = neighbor_cache.parent
    assert parent.shape[0] == output_coords.shape[0]
    C = feats.shape[1]
    unit = max(1, 16 // feats.element_size())
    x = _pad_to(feats.detach().contiguous(), 1, unit)
    out = _ops.sparse_upsample(x, parent.to(torch.int32).contiguous())[:, :C].contiguous()
    out_shape = torch.Size([*tuple(output_shape[: output_coords.shape[1]]), C])
    return out, output_coords, out_shape, neighbor_cache
