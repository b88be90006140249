"""Host-facing mirror of the reference's prompt preparation (promptmoge/model.py:61-72)."""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import ops


def nearest_fill(depth, conf):
    """Drop-in for promptmoge.nearest_fill (promptmoge/model.py:61-72), computed on the GPU.

    Same arguments and results: every pixel with depth <= 0 takes the depth of its nearest valid pixel (exactly
    the pixel scipy.ndimage.distance_transform_edt's index map names) and confidence 1. As in the reference, a
    map that is entirely valid or entirely missing is returned unchanged (the same objects).

    NumPy [h, w] arrays of any dtype come back as NumPy arrays of the same dtypes: the GPU computes the source
    index from the validity mask and the values are gathered from the original arrays, so they are exact.
    GPU tensors [..., h, w] stay on the GPU; fp32 maps are filled in one pass on the device.
    """
    if isinstance(depth, np.ndarray):
        valid = depth > 0
        if valid.all() or not valid.any():
            return depth, conf
        v = torch.from_numpy(np.ascontiguousarray(valid, dtype=np.float32)).to(torch.device("cuda"))
        _, _, idx = ops.nearest_fill(v, None, return_index=True)
        src = idx.cpu().numpy().reshape(-1)
        filled = depth.reshape(-1)[src].reshape(depth.shape)
        return filled, np.where(valid, conf, 1).astype(conf.dtype)
    if depth.dtype == torch.float32 and conf.dtype == torch.float32:
        return ops.nearest_fill(depth.contiguous(), conf.contiguous())
    valid = depth > 0
    h, w = depth.shape[-2:]
    _, _, idx = ops.nearest_fill(valid.float().contiguous(), None, return_index=True)
    flat = depth.reshape(-1, h * w)
    src = idx.reshape(-1, h * w).long().clamp_min(0)
    filled = torch.gather(flat, 1, src).reshape(depth.shape)
    filled = torch.where(idx.reshape(depth.shape) >= 0, filled, depth)
    return filled, torch.where(valid | (idx < 0), conf, torch.ones_like(conf))


def prompt_gauge_poly(depth: torch.Tensor, lidar: torch.Tensor, conf: Optional[torch.Tensor], degree: int = 2,
                      iters: int = 3) -> torch.Tensor:
    """Drop-in for MoGeModel.prompt_gauge_poly (moge/model/v3.py:151-183), computed on the GPU.

    Same arguments and result: depth [B, H, W], lidar / conf [B, 1, h, w] or [B, h, w] (conf may be None); returns
    the [B, H, W] multiplicative correction in depth's dtype. The least squares run in fp64 normal equations (the
    reference: LAPACK on fp32), so the coefficients agree to rounding, not bit for bit.
    """
    corr = ops.gauge_poly(depth.float().contiguous(), lidar.float().contiguous(),
                          None if conf is None else conf.float().contiguous(), degree, iters)
    return corr.to(depth.dtype)
