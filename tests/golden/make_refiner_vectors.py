"""Writes tests/golden/refiner_vectors.npz: input/output vectors of the reference's own refiner modules.

Run once, in the build container only (it needs /root/reference; nothing on the GPU box runs it):

    python tests/golden/make_refiner_vectors.py

It imports, from /root/reference, SparseResBlock3d (moge/model/modules/flex_sparse_blocks.py:50-75),
Sparse3DUNet (moge/model/modules/sparse_unet.py:17-258) and enable_refiner_qat / freeze_observers
(moge/model/modules/qat.py:118-143), over the reference's bundled CPU flex_gemm (promptmoge/_fallback/flex_gemm),
and records, for seeded inputs:

  block.*   one SparseResBlock3d(16) on level-0 voxels of a 2 x 10 x 12 point map: the module's parameters (its own
            seeded initialisation), the input features and the output
  unet.*    a 3-level Sparse3DUNet(3 -> 1, encoder 24, channels [8, 16, 16], encoder blocks [1, 2, 1], decoder
            blocks [2, 1], bottleneck 1, factors [2, 2], prompt channels 2) on a 2 x 16 x 24 point map with
            encoder feature, prompt features and encoder bias map: its state dict (every parameter non-zero), the
            coordinates of every level, per-stage outputs and the output in fp32; then, after enable_refiner_qat
            with frozen activation clips (the 99.95th percentile of |x| of each quantised layer's input in the fp32
            forward), the fake-quantised per-stage outputs and output

These are the only vectors of the refiner's composition the reference can provide (it ships no tests or fixtures
for this path); they pin oracle/unet.py and oracle/refiner.py's block composition (tests/test_oracle_unet.py).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference")
HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path[:0] = [str(REF / "promptmoge" / "_fallback"), str(REF), str(ROOT)]

from moge.model.modules.flex_sparse_blocks import SparseResBlock3d  # noqa: E402
from moge.model.modules.qat import ActFakeQuant, enable_refiner_qat, freeze_observers  # noqa: E402
from moge.model.modules.sparse_unet import Sparse3DUNet  # noqa: E402

from oracle.structure import voxelize  # noqa: E402  (level-0 coordinates, v3.py:327-340)
from promptmoge_amd import spec  # noqa: E402  (seeded synthetic scene)


def level0(B, H, W, seed):
    cfg = spec.StepConfig("g", H, W, 0.9 * W, 0.9 * W, W / 2, H / 2, 16, 1, "int8", seed=seed)
    pts = np.stack([spec.make_scene(cfg, seed=seed + 3 * b).points for b in range(B)])
    zq, coords, zext, _ = voxelize(pts)
    return pts, coords, zext


def randomise(module, gen):
    """Every parameter non-zero (the modules zero-initialise prompt_proj, sparse_unet.py:77-78)."""
    with torch.no_grad():
        for name, p in module.named_parameters():
            if "norm" in name and name.endswith("weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=gen))
            elif p.ndim == 5:
                p.copy_(0.05 * torch.randn(p.shape, generator=gen))
            elif p.ndim == 2:
                p.copy_(torch.randn(p.shape, generator=gen) / np.sqrt(p.shape[1]))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=gen))


def main():
    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(1234)
    out = {}

    # ---- one residual block
    pts, coords, zext = level0(2, 10, 12, seed=31)
    blk = SparseResBlock3d(16)
    randomise(blk, gen)
    feats = torch.randn((coords.shape[0], 16), generator=gen)
    shape = torch.Size([2, 10, 12, zext, 16])
    with torch.no_grad():
        y, _ = blk(feats, torch.from_numpy(coords), shape)
    out["block.coords"], out["block.shape"] = coords, np.array(list(shape), np.int64)
    out["block.feats"], out["block.out"] = feats.numpy(), y.numpy()
    for k, v in blk.state_dict().items():
        out[f"block.sd.{k}"] = v.numpy()

    # ---- a 3-level U-Net
    B, H, W = 2, 16, 24
    pts, coords, zext = level0(B, H, W, seed=41)
    M = coords.shape[0]
    unet = Sparse3DUNet(3, 1, 24, [8, 16, 16], [1, 2, 1], [2, 1], bottleneck_blocks=1, downsample_factors=[2, 2],
                        encoder_downsample=4, prompt_channels=2)
    randomise(unet, gen)
    unet.eval()
    feats = torch.from_numpy(pts.reshape(M, 3))
    enc = torch.randn((B, 24, H // 4, W // 4), generator=gen)
    bias = 0.1 * torch.randn((B, 16, H // 4, W // 4), generator=gen)
    prompt = torch.stack([0.05 * torch.randn(M, generator=gen), torch.rand(M, generator=gen)], 1)
    shape = torch.Size([B, H, W, zext, 3])
    tcoords = torch.from_numpy(coords)

    stages = {}
    hooks = []

    def keep(name, idx=0):
        def hook(mod, args, res):
            stages[name] = (res[idx] if isinstance(res, tuple) else res).detach().clone()
        return hook

    for k, st in enumerate(unet.down_stages):
        hooks.append(st[-1].register_forward_hook(keep(f"down{k}")))
    for k, d in enumerate(unet.downsample_blocks):
        hooks.append(d.register_forward_hook(keep(f"pool{k}")))
        hooks.append(d.register_forward_hook(keep(f"level{k + 1}.coords", 1)))
    hooks.append(unet.encoder_fuse.register_forward_hook(keep("enc_lin")))
    hooks.append(unet.fuse_proj.register_forward_hook(keep("fuse")))
    hooks.append(unet.bottleneck_stage[-1].register_forward_hook(keep("bott")))
    for i, st in enumerate(unet.up_stages):
        hooks.append(st[-1].register_forward_hook(keep(f"dec{i}")))

    # inputs of every layer enable_refiner_qat quantises, for the clips
    seen = {}
    qnames = [n for n, m in unet.named_modules()
              if (type(m).__name__ == "SubmanifoldConv3d" or isinstance(m, torch.nn.Linear))
              and not any(n == s or n.endswith("." + s) for s in ("input_proj", "prompt_proj", "out_proj"))]
    mods = dict(unet.named_modules())
    for n in qnames:
        hooks.append(mods[n].register_forward_pre_hook(
            (lambda name: lambda m, args: seen.__setitem__(name, args[0].detach().clone()))(n)))
    with torch.no_grad():
        y = unet(feats, tcoords, shape, enc, prompt_feats=prompt, encoder_bias_map=bias)
    for h in hooks[-len(qnames):]:
        h.remove()
    hooks = hooks[:-len(qnames)]
    clips = {n: float(torch.quantile(seen[n].abs().flatten().double(), 0.9995)) for n in qnames}

    out["unet.coords"], out["unet.shape"] = coords, np.array(list(shape), np.int64)
    out["unet.feats"], out["unet.enc"], out["unet.bias"] = feats.numpy(), enc.numpy(), bias.numpy()
    out["unet.prompt"], out["unet.out_fp32"] = prompt.numpy(), y.numpy()
    for k, v in stages.items():
        out[f"unet.fp32.{k}"] = v.numpy()
    for k, v in unet.state_dict().items():
        out[f"unet.sd.{k}"] = v.numpy()
    for n, c in clips.items():
        out[f"unet.clip.{n}"] = np.array(c, np.float64)

    # ---- the same U-Net quantisation-aware, clips frozen
    stages.clear()
    enable_refiner_qat(unet)
    for n in qnames:
        aq = getattr(unet, "aq_" + n.replace(".", "_"))
        assert isinstance(aq, ActFakeQuant)
        aq.clip.fill_(clips[n])
        aq.observed.fill_(1)
    freeze_observers(unet)
    unet.eval()
    with torch.no_grad():
        yq = unet(feats, tcoords, shape, enc, prompt_feats=prompt, encoder_bias_map=bias)
    out["unet.out_qat"] = yq.numpy()
    for k, v in stages.items():
        if not k.endswith("coords"):
            out[f"unet.qat.{k}"] = v.numpy()

    path = HERE / "refiner_vectors.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size / 1024:.0f} KiB, {len(out)} arrays)")


if __name__ == "__main__":
    main()
