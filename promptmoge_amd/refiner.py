"""The fused refiner step on the GPU, behind a host object and behind the reference's refiner-module interface.

`RefinerStep` owns a libpmg refiner context (persistent workspace, HIP graph) and runs one refinement step of the
refine loop (moge/model/v3.py:547-576) with no host synchronisation:

    prompt fit (fit_scale_shift)  ->  residual/gate  ->  voxelise  ->  neighbour map  ->  input_proj + prompt_proj
    ->  residual blocks  ->  out_proj  ->  logz += delta            [->  metric fit of the refined depth]

The refined point map (x/z, y/z, logz + delta) is written to `out`, which may be the input itself; that is the
reference loop's `current_coord = cat(xy, refined_logz)` (v3.py:574).

`FusedRefiner` is the refiner module alone, an nn.Module with Sparse3DUNet.forward's signature (the refiner-module
plug point, v3.py:356-357); it runs input_proj -> blocks -> out_proj on given voxel features and returns (M, 1).
"""
from __future__ import annotations

import ctypes as C
from typing import List, Optional

import numpy as np
import torch

from . import _lib
from ._lib import BlockWeights, RefinerConfig, RefinerWeights, call, lib
from .spec import RefinerW, act_mult, act_scale, quantize_weight


class DeviceWeights:
    """A RefinerW uploaded to the GPU in the layouts the kernels read. int8: per-output-channel quantised conv
    weights in the module layout (Co, 3, 3, 3, Ci) with fp32 scales; fp16: fp16 conv weights."""

    def __init__(self, w: RefinerW, precision: str, device="cuda"):
        self.precision = precision
        self.C = w.C
        t = lambda a, dt=torch.float32: torch.as_tensor(np.ascontiguousarray(a)).to(device=device, dtype=dt)
        self.in_w, self.in_b = t(w.in_w), t(w.in_b)
        self.pr_w, self.pr_b = t(w.pr_w), t(w.pr_b)
        self.out_w, self.out_b = t(w.out_w), t(w.out_b)
        self.blocks = []
        for k, b in enumerate(w.blocks):
            d = {"gamma": t(b.gamma), "beta": t(b.beta), "b1": t(b.b1), "b2": t(b.b2)}
            if precision == "int8":
                for name, c in (("conv1", b.clip1), ("conv2", b.clip2)):
                    if not np.isfinite(c) or c <= 0:
                        raise ValueError(f"block {k} {name}: the int8 refiner needs a positive activation clip, "
                                         f"got {c} (a state dict without aq_*.clip entries needs `clips`)")
                q1, s1 = quantize_weight(b.w1)
                q2, s2 = quantize_weight(b.w2)
                d.update(w1=t(q1, torch.int8), s1=t(s1), w2=t(q2, torch.int8), s2=t(s2),
                         a1=float(act_scale(b.clip1)), a2=float(act_scale(b.clip2)),
                         m1=float(act_mult(b.clip1)), m2=float(act_mult(b.clip2)))
            else:
                d.update(w1=t(b.w1, torch.float16), w2=t(b.w2, torch.float16), s1=None, s2=None, a1=1.0, a2=1.0,
                         m1=1.0, m2=1.0)
            self.blocks.append(d)
        self._struct_blocks = (BlockWeights * len(self.blocks))()
        for k, d in enumerate(self.blocks):
            p = lambda x: None if x is None else x.data_ptr()
            self._struct_blocks[k] = BlockWeights(
                p(d["gamma"]), p(d["beta"]), p(d["w1"]), p(d["s1"]), p(d["b1"]), d["a1"], d["m1"],
                p(d["w2"]), p(d["s2"]), p(d["b2"]), d["a2"], d["m2"])
        self.struct = RefinerWeights(
            self.in_w.data_ptr(), self.in_b.data_ptr(), self.pr_w.data_ptr(), self.pr_b.data_ptr(),
            self.out_w.data_ptr(), self.out_b.data_ptr(), len(self.blocks),
            C.cast(self._struct_blocks, C.POINTER(BlockWeights)))


class RefinerStep:
    """One fused refinement step for point maps of a fixed size.

    points [B, H, W, 3] fp32 (x/z, y/z, logz) is refined into `out` (default in place); lidar, conf [B, dh, dw].
    Returns the prompt fit (s, t) [B, 2] and, if `final_fit`, the metric fit of the refined depth [B, 2].
    `output_gate` / `output_gate_floor` and `anchor` are the refine loop's lidar_prompt options 'output_gate',
    'output_gate_floor' and 'anchor' (v3.py:40-41, 565-573). With `post_depth` (and `final_fit`) every call also
    writes the metric depth s * exp(logz) + t of the refined map into `self.depth` [B, H, W] (+inf where not > 0;
    MetricFit.metal:200-211).
    """

    def __init__(self, weights: RefinerW, B: int, H: int, W: int, dh: Optional[int] = None,
                 dw: Optional[int] = None, *, precision: str = "int8", depth_resolution: float = 256.0,
                 fit_iters: int = 4, fit_trim: float = 0.2, fit_min_points: int = 32, use_prompt: bool = True,
                 soft_gate: bool = False, final_fit: bool = False, use_graph: bool = True,
                 output_gate: bool = False, output_gate_floor: float = 0.1, anchor: float = 0.0,
                 post_depth: bool = False, device="cuda"):
        if precision not in ("int8", "fp16"):
            raise ValueError("precision must be 'int8' or 'fp16'")
        if post_depth and not final_fit:
            raise ValueError("post_depth needs final_fit")
        self.post_depth = post_depth
        self.depth = torch.empty((B, H, W), dtype=torch.float32, device=device) if post_depth else None
        self.B, self.H, self.W = B, H, W
        self.dh, self.dw = dh or H, dw or W
        self.final_fit = final_fit
        self.weights = DeviceWeights(weights, precision, device)
        cfg = RefinerConfig(B, H, W, weights.C, len(weights.blocks),
                            _lib.PREC_INT8 if precision == "int8" else _lib.PREC_FP16, float(depth_resolution),
                            self.dh, self.dw, int(fit_iters), float(fit_trim), int(fit_min_points), int(use_prompt),
                            int(soft_gate), int(final_fit), int(use_graph), int(output_gate),
                            float(output_gate_floor), float(anchor))
        self._h = lib().pmg_refiner_create(C.byref(cfg))
        if not self._h:
            raise _lib.PmgError(_lib.PMG_E_INVALID, lib().pmg_last_error().decode())
        call("pmg_refiner_set_weights", self._h, C.byref(self.weights.struct))
        self.st_prompt = torch.zeros((B, 2), dtype=torch.float32, device=device)
        self.st_final = torch.zeros((B, 2), dtype=torch.float32, device=device)

    def close(self) -> None:
        """Releases the device workspace and graphs (also done when the object is collected)."""
        h = getattr(self, "_h", None)
        if h:
            self._h = None
            lib().pmg_refiner_destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library handle may already be gone
            pass

    def __call__(self, points: torch.Tensor, lidar: torch.Tensor, conf: torch.Tensor,
                 out: Optional[torch.Tensor] = None):
        """Refines `points` into `out` (default: in place). Returns (st_prompt [B, 2], st_final [B, 2] | None)."""
        out = points if out is None else out
        for name, t in (("points", points), ("out", out)):
            if t.shape != (self.B, self.H, self.W, 3) or t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous fp32 [{self.B}, {self.H}, {self.W}, 3] tensor")
        for name, t in (("lidar", lidar), ("conf", conf)):
            if t.shape != (self.B, self.dh, self.dw) or t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous fp32 [{self.B}, {self.dh}, {self.dw}] tensor")
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        call("pmg_refiner_step", self._h, points.data_ptr(), out.data_ptr(), lidar.data_ptr(), conf.data_ptr(),
             self.st_prompt.data_ptr(), self.st_final.data_ptr() if self.final_fit else None, stream)
        if self.post_depth:  # the metric depth of the refined map, MetricFit.metal:200-211 (self.depth)
            call("pmg_post_depth", out.data_ptr() + 8, 3, None, self.B, self.H, self.W, self.st_final.data_ptr(),
                 self.depth.data_ptr(), stream)
        return self.st_prompt, (self.st_final if self.final_fit else None)

    def check(self) -> None:
        """Synchronises and raises if a device-side bounded wait expired."""
        call("pmg_refiner_check", self._h, C.c_void_p(torch.cuda.current_stream().cuda_stream))

    def buffer(self, which: str) -> torch.Tensor:
        """A copy of an internal buffer of the last step (parity tests): zq (voxel keys), x (residual entering the
        last block), q1 / q2 (the last block's conv1 / conv2 input)."""
        ids = {"zq": 0, "x": 3, "q1": 4, "q2": 5}
        M, Cc = self.B * self.H * self.W, self.weights.C
        f16 = self.weights.precision == "fp16"
        shape, dt = {
            "zq": ((M,), torch.int32),
            "x": ((M, Cc), torch.float32), "q1": ((M, Cc), torch.float16 if f16 else torch.int8),
            "q2": ((M, Cc), torch.float16 if f16 else torch.int8),
        }[which]
        ptr = lib().pmg_refiner_buffer(self._h, ids[which])
        out = torch.empty(shape, dtype=dt, device=self.st_prompt.device)
        nbytes = out.numel() * out.element_size()
        _copy_device(out.data_ptr(), ptr, nbytes, torch.cuda.current_stream().cuda_stream)
        return out


def _copy_device(dst: int, src: int, nbytes: int, stream: int) -> None:
    """Device-to-device copy of a raw buffer, ordered on `stream` (the stream torch uses next), through the HIP
    runtime torch already loaded. A plain hipMemcpy would not do: device-to-device it may return before the copy
    is done, and it runs on the null stream, which torch's streams do not wait for."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpyAsync.restype = C.c_int
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    rc = hip.hipMemcpyAsync(C.c_void_p(dst), C.c_void_p(src), C.c_size_t(nbytes), 3, C.c_void_p(stream))
    if rc != 0:
        raise RuntimeError(f"hipMemcpyAsync failed with {rc}")


class FusedRefiner(torch.nn.Module):
    """The refiner module on the GPU, behind Sparse3DUNet.forward's signature (moge/model/modules/sparse_unet.py:
    176-258): `forward(feats, coords, shape, encoder_feature, prompt_feats=None, encoder_bias_map=None) -> (M, 1)`,
    what `_refine_logz` calls at v3.py:356-357 (`model.refiner = FusedRefiner(...)`, or `refiner=` there).

    The network is the single-level refiner: input_proj (3 -> C) + prompt_proj (2 -> C) of the given prompt
    features, n_blocks SparseResBlock3d(C) (flex_sparse_blocks.py:50-75) in the deployed int8 contract (or the fp16
    teacher), out_proj (C -> 1). The voxels must be level 0 as _voxelize builds them (v3.py:305-344): one per
    pixel in raster (b, i, j) order, so the neighbour map is the column stencil on coords[:, 3] and is never
    materialised. `encoder_feature` and `encoder_bias_map` feed the multi-level U-Net's bottleneck fusion, which
    a single-level refiner does not have; they are accepted and not read. Inference only.
    """

    def __init__(self, weights: RefinerW, *, precision: str = "int8", depth_resolution: float = 256.0,
                 use_graph: bool = True, check_coords: bool = True):
        super().__init__()
        if precision not in ("int8", "fp16"):
            raise ValueError("precision must be 'int8' or 'fp16'")
        self.host_weights = weights
        self.precision = precision
        self.depth_resolution = float(depth_resolution)
        self.use_graph = use_graph
        self.check_coords = check_coords
        self._weights = {}   # device -> DeviceWeights
        self._ctx = {}       # (device, B, H, W) -> refiner handle
        self._io = {}        # (device, B, H, W) -> persistent input / output buffers of that context

    def _handle(self, device: torch.device, B: int, H: int, W: int):
        key = (device.index, B, H, W)
        h = self._ctx.get(key)
        if h is None:
            dw = self._weights.get(device.index)
            if dw is None:
                dw = self._weights[device.index] = DeviceWeights(self.host_weights, self.precision, device)
            w = self.host_weights
            cfg = RefinerConfig(B, H, W, w.C, len(w.blocks),
                                _lib.PREC_INT8 if self.precision == "int8" else _lib.PREC_FP16,
                                self.depth_resolution, H, W, 0, 0.2, 32, 1, 0, 0, int(self.use_graph))
            h = lib().pmg_refiner_create(C.byref(cfg))
            if not h:
                raise _lib.PmgError(_lib.PMG_E_INVALID, lib().pmg_last_error().decode())
            call("pmg_refiner_set_weights", h, C.byref(dw.struct))
            self._ctx[key] = h
            M = B * H * W
            dev = torch.device("cuda", device.index)
            self._io[key] = {
                "feats": torch.empty((M, 3), dtype=torch.float32, device=dev),
                "coords": torch.empty((M, 4), dtype=torch.int32, device=dev),
                "prompt": torch.empty((M, 2), dtype=torch.float32, device=dev),
                "out": torch.empty((M,), dtype=torch.float32, device=dev),
            }
        return h

    def forward(self, feats: torch.Tensor, coords: Optional[torch.Tensor], shape, encoder_feature=None,
                prompt_feats: Optional[torch.Tensor] = None, encoder_bias_map=None) -> torch.Tensor:
        if torch.is_grad_enabled() and feats.requires_grad:
            raise NotImplementedError("FusedRefiner is inference-only")
        B, H, W = int(shape[0]), int(shape[1]), int(shape[2])
        M = B * H * W
        if feats.shape != (M, 3) or not feats.is_cuda:
            raise ValueError(f"feats must be a GPU tensor (M, 3) with M = B*H*W = {M} (level-0 voxels)")
        feats = feats.float().contiguous()
        if coords is not None:
            coords = coords.to(torch.int32).contiguous()
            if coords.shape != (M, 4):
                raise ValueError("coords must be (M, 4)")
            if self.check_coords and not _is_raster(coords, B, H, W):
                raise ValueError("coords are not level-0 raster order (one voxel per pixel, _voxelize)")
        if prompt_feats is not None:
            prompt_feats = prompt_feats.float().contiguous()
            if prompt_feats.shape != (M, 2):
                raise ValueError("prompt_feats must be (M, 2)")
        h = self._handle(feats.device, B, H, W)
        # The context replays one captured graph per (buffers, stream). The inputs are staged into the context's
        # persistent buffers (a few MB of device copies on the same stream), so every call replays the same graph
        # instead of capturing a new one for each fresh tensor; the result is copied out, so the caller owns it.
        io = self._io[(feats.device.index, B, H, W)]
        io["feats"].copy_(feats)
        if coords is not None:
            io["coords"].copy_(coords)
        if prompt_feats is not None:
            io["prompt"].copy_(prompt_feats)
        call("pmg_refiner_forward", h, io["feats"].data_ptr(), io["coords"].data_ptr() if coords is not None else None,
             io["prompt"].data_ptr() if prompt_feats is not None else None, io["out"].data_ptr(),
             C.c_void_p(torch.cuda.current_stream().cuda_stream))
        return io["out"].clone().view(M, 1)

    def close(self) -> None:
        for h in self._ctx.values():
            lib().pmg_refiner_destroy(h)
        self._ctx.clear()
        self._io.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library handle may already be gone
            pass


def _is_raster(coords: torch.Tensor, B: int, H: int, W: int) -> bool:
    """coords[:, :3] == (b, i, j) in raster order, the test of _is_one_voxel_per_column (_core.py:249-266)."""
    m = torch.arange(B * H * W, device=coords.device, dtype=torch.int32)
    ref = torch.stack([m // (H * W), (m // W) % H, m % W], dim=1)
    return bool(torch.equal(coords[:, :3], ref))
