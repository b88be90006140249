"""The multi-level refiner on the GPU (int8, or the fp16 teacher), behind Sparse3DUNet.forward's signature.

`UNetRefiner` is an nn.Module with the forward of Sparse3DUNet (moge/model/modules/sparse_unet.py:176-258),
`forward(feats, coords, shape, encoder_feature, prompt_feats=None, encoder_bias_map=None) -> (M, 1)`, the call
`_refine_logz` makes (v3.py:356-357): `model.refiner = UNetRefiner.from_state_dict(model.refiner.state_dict())`
(or `refiner=` there). It runs the whole U-Net -- level structure, per-level maps, int8 convolutions and linears,
encoder conditioning -- in libpmg (`pmg_unet_*`, csrc/pmg_unet.hip) as one captured HIP graph with no host
synchronisation. The voxels must be level 0 as _voxelize builds them (v3.py:305-344): one per pixel in raster order.

`UNetStep` is one whole refine-loop step with that refiner (v3.py:547-576): prompt fit, (residual, gate) prompt
features, _voxelize, the U-Net, logz + delta (output gate), elastic anchor, final metric fit and post_depth, one
captured graph on the device (`pmg_unet_step`), with no host round trip between them.

Weights come from a Sparse3DUNet state dict (plain or QAT), from the Metal engine's refiner.bin / refiner.json
export, or from promptmoge_amd.unet_weights.make_unet_weights; the arithmetic is the deployed int8 contract
(qat.py:1-16): per-output-channel int8 weights, per-tensor int8 activations with the layer's clip, int32
accumulation -- or, with precision="fp16", the teacher's (PromptMoGe-L, e.g. the stock 32 64 128 256 512 refiner,
train.py:124): fp16 activations and weights in every convolution and linear, fp32 accumulation, fp32 residual
streams, LayerNorm and SiLU in fp32. Inference only.
"""
from __future__ import annotations

import ctypes as C
from typing import Dict, Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import BlockWeights, LinearWeights, UNetConfig, UNetStepConfig, UNetWeights, call, lib
from .spec import act_mult, act_scale
from .unet_weights import UNetW, load_refiner_bin, quantized, unet_from_state_dict


class UNetDeviceWeights:
    """A UNetW on the GPU in the layouts the kernels read: conv weights int8 (Co, 3, 3, 3, Ci), linear weights int8
    (N, K), per-output-channel fp32 scales, fp32 biases / LayerNorm affine, activation scales from the clips; with
    precision "fp16" (the teacher) the conv and linear weights in fp16 and no scales or clips."""

    def __init__(self, w: UNetW, device, precision: str = "int8"):
        t = lambda a, dt=torch.float32: torch.as_tensor(np.ascontiguousarray(a)).to(device=device, dtype=dt)
        self.keep = []

        def dev(a, dt=torch.float32):
            x = t(a, dt)
            self.keep.append(x)
            return x.data_ptr()

        self.in_w, self.in_b = dev(w.in_w), dev(w.in_b)
        self.pr_w = dev(w.pr_w) if w.pr_w is not None else None
        self.pr_b = dev(w.pr_b) if w.pr_b is not None else None
        self.out_w, self.out_b = dev(np.asarray(w.out_w).reshape(-1)), dev(np.asarray(w.out_b).reshape(-1))
        blocks = [b for st in w.down for b in st] + list(w.bott) + [b for st in w.dec for b in st]
        self._blocks = (BlockWeights * max(len(blocks), 1))()
        f16 = precision == "fp16"
        h = lambda a: dev(np.asarray(a, np.float32), torch.float16)
        for k, b in enumerate(blocks):
            if f16:
                self._blocks[k] = BlockWeights(dev(b.gamma), dev(b.beta), h(b.w1), None, dev(b.b1), 1.0, 1.0, h(b.w2),
                                               None, dev(b.b2), 1.0, 1.0)
                continue
            q1, s1 = quantized(b.w1)
            q2, s2 = quantized(b.w2)
            self._blocks[k] = BlockWeights(
                dev(b.gamma), dev(b.beta), dev(q1, torch.int8), dev(s1), dev(b.b1), float(act_scale(b.clip1)),
                float(act_mult(b.clip1)), dev(q2, torch.int8), dev(s2), dev(b.b2), float(act_scale(b.clip2)),
                float(act_mult(b.clip2)))
        linears = list(w.pool) + [w.enc, w.fuse0, w.fuse2] + list(w.up)
        self._linears = (LinearWeights * len(linears))()
        for k, l in enumerate(linears):
            if f16:
                self._linears[k] = LinearWeights(h(l.w), None, dev(l.b), 1.0, 1.0)
                continue
            q, s = quantized(l.w)
            self._linears[k] = LinearWeights(dev(q, torch.int8), dev(s), dev(l.b), float(act_scale(l.clip)),
                                             float(act_mult(l.clip)))
        self.struct = UNetWeights(self.in_w, self.in_b, self.pr_w, self.pr_b, self.out_w, self.out_b, len(blocks),
                                  C.cast(self._blocks, C.POINTER(BlockWeights)), len(linears),
                                  C.cast(self._linears, C.POINTER(LinearWeights)))


class UNetRefiner(torch.nn.Module):
    """Sparse3DUNet on the GPU in the deployed int8 arithmetic, or (precision="fp16") in the teacher's half
    precision (see the module docstring)."""

    def __init__(self, weights: UNetW, *, depth_resolution: float = 256.0, use_graph: bool = True,
                 check_coords: bool = True, precision: str = "int8"):
        super().__init__()
        if any(f != 2 for f in weights.factors):
            raise ValueError("downsample factors other than 2 are not supported (MoGe's refiners use 2)")
        if precision not in ("int8", "fp16"):
            raise ValueError("precision must be 'int8' or 'fp16'")
        if precision == "int8":
            wide = [c for c in weights.channels if c not in (16, 32, 48, 64, 96, 128, 192, 256)]
            if wide or weights.channels[0] not in (16, 32, 48, 64, 128):
                # the deployed int8 refiners are the narrowed 32 64 128 256 256 (train.py:124); the stock 512-wide
                # refiner is the teacher, which runs in fp16 (precision="fp16")
                raise ValueError(f"UNetRefiner (int8) takes level widths 16, 32, 48, 64, 96, 128, 192, 256 (level 0: "
                                 f"16, 32, 48, 64, 128); got {weights.channels}")
        else:
            wide = [c for c in weights.channels if c not in (16, 32, 48, 64, 96, 128, 192, 256, 512)]
            if wide or weights.channels[0] not in (16, 32, 48, 64):
                raise ValueError(f"UNetRefiner (fp16) takes level widths 16, 32, 48, 64, 96, 128, 192, 256, 512 "
                                 f"(level 0: 16, 32, 48, 64); got {weights.channels}")
        self.precision = precision
        self.host_weights = weights
        self.depth_resolution = float(depth_resolution)
        self.use_graph = use_graph
        self.check_coords = check_coords
        self._weights: Dict[int, UNetDeviceWeights] = {}
        self._ctx: Dict[tuple, int] = {}
        self._io: Dict[tuple, dict] = {}
        self._last_key: Dict[tuple, Optional[tuple]] = {}  # per context: the previous call's input buffers

    @classmethod
    def from_state_dict(cls, sd, factors: Optional[Sequence[int]] = None, clips=None, **kw) -> "UNetRefiner":
        """From a Sparse3DUNet state dict (unet_weights.unet_from_state_dict): QAT, or plain with `clips`; with
        precision="fp16" (the teacher) any plain state dict, no clips needed."""
        f16 = kw.get("precision", "int8") == "fp16"
        return cls(unet_from_state_dict(sd, factors, clips, require_clips=not f16), **kw)

    @classmethod
    def from_refiner_bin(cls, directory, **kw):
        """From the Metal engine's refiner.bin / refiner.json (promptmoge/export/refiner.py:28-110). Returns
        (module, uv_bias [C_L, R, C] or None): uv_bias is the encoder bias map of every frame of that grid."""
        w, man, uv = load_refiner_bin(directory)
        return cls(w, depth_resolution=float(man.get("depth_resolution", 256.0)), **kw), uv

    def _config(self, B: int, H: int, W: int) -> UNetConfig:
        w = self.host_weights
        L = w.levels
        pad = lambda xs: (_lib.i32 * 8)(*(list(xs) + [0] * (8 - len(xs))))
        return UNetConfig(B, H, W, L, pad(w.channels), pad([len(s) for s in w.down]), pad([len(s) for s in w.dec]),
                          len(w.bott), int(w.enc_channels), self.depth_resolution, int(self.use_graph),
                          _lib.PREC_FP16 if self.precision == "fp16" else _lib.PREC_INT8)

    def _handle(self, device: torch.device, B: int, H: int, W: int):
        key = (device.index, B, H, W)
        h = self._ctx.get(key)
        if h is None:
            dw = self._weights.get(device.index)
            if dw is None:
                dw = self._weights[device.index] = UNetDeviceWeights(self.host_weights, device, self.precision)
            cfg = self._config(B, H, W)
            h = lib().pmg_unet_create(C.byref(cfg))
            if not h:
                raise _lib.PmgError(_lib.PMG_E_INVALID, lib().pmg_last_error().decode())
            call("pmg_unet_set_weights", h, C.byref(dw.struct))
            self._ctx[key] = h
            M = B * H * W
            w = self.host_weights
            ds = 2 ** (w.levels - 1)
            dev = torch.device("cuda", device.index)
            self._io[key] = {
                "feats": torch.empty((M, 3), dtype=torch.float32, device=dev),
                "coords": torch.empty((M, 4), dtype=torch.int32, device=dev),
                "prompt": torch.empty((M, 2), dtype=torch.float32, device=dev),
                "enc": torch.empty((B, w.enc_channels, H // ds, W // ds), dtype=torch.float32, device=dev),
                "bias": torch.empty((B, w.channels[-1], H // ds, W // ds), dtype=torch.float32, device=dev),
                "out": torch.empty((M,), dtype=torch.float32, device=dev),
            }
        return h

    def forward(self, feats: torch.Tensor, coords: Optional[torch.Tensor], shape, encoder_feature: torch.Tensor,
                prompt_feats: Optional[torch.Tensor] = None,
                encoder_bias_map: Optional[torch.Tensor] = None) -> torch.Tensor:
        if torch.is_grad_enabled() and feats.requires_grad:
            raise NotImplementedError("UNetRefiner is inference-only")
        w = self.host_weights
        B, H, W = int(shape[0]), int(shape[1]), int(shape[2])
        M = B * H * W
        ds = 2 ** (w.levels - 1)
        if feats.shape != (M, 3) or not feats.is_cuda:
            raise ValueError(f"feats must be a GPU tensor (M, 3) with M = B*H*W = {M} (level-0 voxels)")
        # sparse_unet.py:185-187: the point map is encoder_downsample times the encoder grid
        if encoder_feature.ndim != 4 or encoder_feature.shape[0] != B or encoder_feature.shape[1] != w.enc_channels \
                or H != encoder_feature.shape[2] * ds or W != encoder_feature.shape[3] * ds:
            raise ValueError(f"encoder_feature must be [B, {w.enc_channels}, H/{ds}, W/{ds}]")
        if coords is not None:
            coords = coords.to(torch.int32)
            if coords.shape != (M, 4):
                raise ValueError("coords must be (M, 4)")
            if self.check_coords and not _is_raster(coords, B, H, W):
                raise ValueError("coords are not level-0 raster order (one voxel per pixel, _voxelize)")
        if prompt_feats is not None and prompt_feats.shape != (M, 2):
            raise ValueError("prompt_feats must be (M, 2)")
        if encoder_bias_map is not None and encoder_bias_map.shape != (B, w.channels[-1], H // ds, W // ds):
            raise ValueError(f"encoder_bias_map must be [B, {w.channels[-1]}, H/{ds}, W/{ds}]")
        h = self._handle(feats.device, B, H, W)
        ctx = (feats.device.index, B, H, W)
        io = self._io[ctx]
        # The library replays one captured graph per set of input buffers. A caller that passes the same tensors
        # as in its previous call (contiguous, fp32 / int32, 16-byte aligned) has them read in place: its graph is
        # captured once and replayed with no copies. Other inputs are staged into the context's persistent
        # buffers, whose graph is always cached, so varying tensors never cost a capture.
        given = {"feats": feats, "coords": coords, "prompt": prompt_feats, "enc": encoder_feature,
                 "bias": encoder_bias_map}
        usable = all(t is None or (t.is_contiguous() and t.device == feats.device and t.data_ptr() % 16 == 0
                                   and t.dtype == io[n].dtype) for n, t in given.items())
        key = tuple(None if t is None else t.data_ptr() for t in given.values())
        direct = usable and self._last_key.get(ctx) == key
        self._last_key[ctx] = key if usable else None
        src = {}
        for n, t in given.items():
            if t is None:
                src[n] = None
            elif direct:
                src[n] = t.data_ptr()
            else:
                io[n].copy_(t)
                src[n] = io[n].data_ptr()
        call("pmg_unet_forward", h, src["feats"], src["coords"], src["prompt"], src["enc"], src["bias"],
             io["out"].data_ptr(), C.c_void_p(torch.cuda.current_stream().cuda_stream))
        return io["out"].clone().view(M, 1)

    def buffer(self, which: str, level: int, shape=None) -> torch.Tensor:
        """A copy of a device buffer of the last forward (parity tests): counts, coords, parent, nmap, tile_mask,
        col_offsets, down, up, enc_tokens (see pmg_unet_buffer)."""
        if len(self._ctx) != 1:
            raise RuntimeError("buffer() needs exactly one context")
        key, h = next(iter(self._ctx.items()))
        B, H, W = key[1:]
        w = self.host_weights
        cap = B * H * W
        ids = {"counts": (_lib.UNET_COUNTS, (w.levels,), torch.int64),
               "coords": (_lib.UNET_COORDS, (cap, 4), torch.int32),
               "parent": (_lib.UNET_PARENT, (cap,), torch.int32),
               "nmap": (_lib.UNET_NMAP, (27, cap), torch.int32),
               "tile_mask": (_lib.UNET_TILE_MASK, ((cap + 15) // 16,), torch.int32),
               "down": (_lib.UNET_DOWN, (cap, w.channels[level]), torch.float32),
               "up": (_lib.UNET_UP, (cap, w.channels[level]), torch.float32),
               "enc_tokens": (_lib.UNET_ENC_TOKENS,
                              (B * (H >> (w.levels - 1)) * (W >> (w.levels - 1)), w.channels[-1]), torch.float32)}
        if which == "col_offsets":
            n = B * -(-H // 2 ** level) * -(-W // 2 ** level) + 1
            ids["col_offsets"] = (_lib.UNET_COL_OFFSETS, (n,), torch.int32)
        bid, shp, dt = ids[which]
        ptr = lib().pmg_unet_buffer(h, bid, level)
        if not ptr:
            raise ValueError(f"level {level} has no {which}")
        out = torch.empty(shape or shp, dtype=dt, device=torch.device("cuda", key[0]))
        from .refiner import _copy_device

        _copy_device(out.data_ptr(), ptr, out.numel() * out.element_size(), torch.cuda.current_stream().cuda_stream)
        return out

    def close(self) -> None:
        for h in self._ctx.values():
            lib().pmg_unet_destroy(h)
        self._ctx.clear()
        self._io.clear()
        self._last_key.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library handle may already be gone
            pass


class UNetStep:
    """One refine-loop step with the multi-level refiner (int8, or the fp16 teacher), fused on the GPU
    (pmg_unet_step).

    points [B, H, W, 3] fp32 (x/z, y/z, logz) is refined into `out` (default in place); lidar, conf [B, dh, dw];
    encoder_feature [B, C_enc, H/ds, W/ds] and encoder_bias_map [B, C_{L-1}, H/ds, W/ds] (or None) as for
    Sparse3DUNet.forward. Returns the prompt fit (s, t) [B, 2] (None without the prompt) and, with `final_fit`, the
    metric fit of the refined depth [B, 2]. The options are the refine loop's: `use_prompt` (use_refiner_residual,
    v3.py:548-555) with `soft_gate`, `output_gate` / `output_gate_floor` and `anchor` (v3.py:565-573), `fit_iters`,
    `fit_trim`, `fit_min_points` (fit_scale_shift's); with `post_depth` (and `final_fit`) every call also writes
    s * exp(logz) + t of the refined map into `self.depth` [B, H, W] (+inf where not > 0; MetricFit.metal:200-211).
    Inference only; the step allocates nothing after construction.
    """

    def __init__(self, weights, B: int, H: int, W: int, dh: Optional[int] = None, dw: Optional[int] = None, *,
                 depth_resolution: float = 256.0, precision: str = "int8", fit_iters: int = 4, fit_trim: float = 0.2, fit_min_points: int = 32,
                 use_prompt: bool = True, soft_gate: bool = False, output_gate: bool = False,
                 output_gate_floor: float = 0.1, anchor: float = 0.0, final_fit: bool = False,
                 post_depth: bool = False, use_graph: bool = True, device="cuda"):
        mod = weights if isinstance(weights, UNetRefiner) else UNetRefiner(weights, depth_resolution=depth_resolution,
                                                                           precision=precision)
        w = mod.host_weights
        if post_depth and not final_fit:
            raise ValueError("post_depth needs final_fit")
        if use_prompt and w.pr_w is None:
            raise ValueError("use_prompt needs a refiner with prompt_proj")
        ds = 2 ** (w.levels - 1)
        if H % ds or W % ds:
            raise ValueError(f"H and W must be multiples of the encoder downsampling {ds} (sparse_unet.py:187)")
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.B, self.H, self.W = B, H, W
        self.dh, self.dw = dh or H, dw or W
        self.use_prompt, self.final_fit, self.post_depth = use_prompt, final_fit, post_depth
        self.host_weights = w
        self.weights = UNetDeviceWeights(w, self.device, mod.precision)
        pad = lambda xs: (_lib.i32 * 8)(*(list(xs) + [0] * (8 - len(xs))))
        cfg = UNetConfig(B, H, W, w.levels, pad(w.channels), pad([len(st) for st in w.down]),
                         pad([len(st) for st in w.dec]), len(w.bott), int(w.enc_channels), float(mod.depth_resolution),
                         int(use_graph), _lib.PREC_FP16 if mod.precision == "fp16" else _lib.PREC_INT8)
        with torch.cuda.device(self.device):
            self.h = lib().pmg_unet_create(C.byref(cfg))
            if not self.h:
                raise _lib.PmgError(_lib.PMG_E_INVALID, lib().pmg_last_error().decode())
            call("pmg_unet_set_weights", self.h, C.byref(self.weights.struct))
            scfg = UNetStepConfig(self.dh, self.dw, int(fit_iters), float(fit_trim), int(fit_min_points),
                                  int(use_prompt), int(soft_gate), int(output_gate), float(output_gate_floor),
                                  float(anchor), int(final_fit))
            call("pmg_unet_step_prepare", self.h, C.byref(scfg))
        self.st_prompt = torch.zeros((B, 2), dtype=torch.float32, device=self.device)
        self.st_final = torch.zeros((B, 2), dtype=torch.float32, device=self.device)
        self.depth = torch.empty((B, H, W), dtype=torch.float32, device=self.device) if post_depth else None

    def __call__(self, points: torch.Tensor, lidar: torch.Tensor, conf: torch.Tensor, encoder_feature: torch.Tensor,
                 encoder_bias_map: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
        w = self.host_weights
        B, H, W = self.B, self.H, self.W
        ds = 2 ** (w.levels - 1)
        need = lambda t, shape, name: _need(t, shape, name, self.device)
        need(points, (B, H, W, 3), "points")
        need(lidar, (B, self.dh, self.dw), "lidar")
        need(conf, (B, self.dh, self.dw), "conf")
        need(encoder_feature, (B, w.enc_channels, H // ds, W // ds), "encoder_feature")
        if encoder_bias_map is not None:
            need(encoder_bias_map, (B, w.channels[-1], H // ds, W // ds), "encoder_bias_map")
        out = points if out is None else out
        need(out, (B, H, W, 3), "out")
        p = lambda t: None if t is None else t.data_ptr()
        call("pmg_unet_step", self.h, points.data_ptr(), out.data_ptr(), lidar.data_ptr(), conf.data_ptr(),
             encoder_feature.data_ptr(), p(encoder_bias_map), self.st_prompt.data_ptr(), self.st_final.data_ptr(),
             p(self.depth), C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream))
        return (self.st_prompt if self.use_prompt else None), (self.st_final if self.final_fit else None)

    def anchor_fit(self) -> torch.Tensor:
        """A copy of the last step's anchor re-fit (s, t) [B, 2] (for parity tests)."""
        ptr = lib().pmg_unet_buffer(self.h, _lib.UNET_STEP_ST, 0)
        out = torch.empty((self.B, 2), dtype=torch.float32, device=self.device)
        from .refiner import _copy_device

        _copy_device(out.data_ptr(), ptr + 4 * 4 * self.B, 8 * self.B,
                     torch.cuda.current_stream(self.device).cuda_stream)
        return out

    def check(self) -> None:
        """Synchronises the stream; raises if a metric fit's device-wide wait expired in a step since the last
        check."""
        call("pmg_unet_check", self.h, C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().pmg_unet_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library handle may already be gone
            pass


def _need(t: torch.Tensor, shape, name: str, device: torch.device) -> None:
    if t.dtype != torch.float32 or tuple(t.shape) != tuple(shape) or not t.is_contiguous() or t.device != device:
        raise ValueError(f"{name} must be a contiguous float32 tensor {tuple(shape)} on {device}, got "
                         f"{t.dtype} {tuple(t.shape)} on {t.device}")


def _is_raster(coords: torch.Tensor, B: int, H: int, W: int) -> bool:
    """coords[:, :3] == (b, i, j) in raster order, the test of _is_one_voxel_per_column (_core.py:249-266)."""
    m = torch.arange(B * H * W, device=coords.device, dtype=torch.int32)
    ref = torch.stack([m // (H * W), (m // W) % H, m % W], dim=1)
    return bool(torch.equal(coords[:, :3], ref))
