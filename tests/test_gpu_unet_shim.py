"""A multi-level sparse U-Net run through the flex_gemm shim against an fp64 restatement.

The network is the sparse part of the reference's Sparse3DUNet.forward (moge/model/modules/sparse_unet.py:176-258):
input_proj -> per level a SparseResBlock3d (flex_sparse_blocks.py:50-75) -> PoolDown (flex_sparse_blocks.py:78-90:
mean pool by 2, then Linear) ... bottleneck block ... NearestUp (flex_sparse_blocks.py:93-105: Linear, then nearest
upsampling with the transposed pool cache) + skip -> block -> out_proj, with the per-level conv caches and the
.T pool caches reused exactly as sparse_unet.py:208-256 reuses them. Sparse operators are the shim's (GPU maps,
fp32 MFMA convs, GPU pooling/upsampling); the dense layers are torch's. The check is oracle/ (conv in the
_fallback per-tap order, sorted / column maps, pool cache, mean pool, upsample) in fp64: the fp32 GPU result must
agree within 2e-5 of the output's magnitude (fp32 accumulation in another order). Encoder conditioning
(encoder_fuse / fuse_proj) is not part of this network."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from oracle import conv as ocv
from oracle import pool as opl
from oracle import structure as ost
from promptmoge_amd import flex_gemm as fg
from promptmoge_amd import spec

from conftest import announce

pytestmark = pytest.mark.gpu


class Block(nn.Module):
    """SparseResBlock3d (flex_sparse_blocks.py:50-75): h = SiLU(LN(x)); conv1; SiLU; conv2; + x."""

    def __init__(self, C):
        super().__init__()
        self.norm1 = nn.LayerNorm(C, eps=1e-6)
        self.conv1 = fg.nn.SubmanifoldConv3d(C, C, 3)
        self.conv2 = fg.nn.SubmanifoldConv3d(C, C, 3)

    def forward(self, x, coords, shape, cache=None):
        h = F.silu(self.norm1(x))
        h, cache = self.conv1(h, coords, shape, neighbor_cache=cache)
        h = F.silu(h)
        h, cache = self.conv2(h, coords, shape, neighbor_cache=cache)
        return h + x, cache


class UNet(nn.Module):
    def __init__(self, chans=(16, 32, 48)):
        super().__init__()
        self.chans = chans
        self.input_proj = nn.Linear(3, chans[0])
        self.down = nn.ModuleList([Block(c) for c in chans])
        self.pool = nn.ModuleList([fg.nn.SparsePool3d(2) for _ in chans[:-1]])
        self.pool_lin = nn.ModuleList([nn.Linear(a, b) for a, b in zip(chans[:-1], chans[1:])])
        self.bottleneck = Block(chans[-1])
        self.up = nn.ModuleList([fg.nn.SparseUpsample3d(2) for _ in chans[:-1]])
        self.up_lin = nn.ModuleList([nn.Linear(b, a) for a, b in zip(chans[:-1], chans[1:])])
        self.up_blocks = nn.ModuleList([Block(c) for c in chans[:-1]])
        self.out_proj = nn.Linear(chans[0], 1)
        with torch.no_grad():
            for p in self.parameters():
                p.normal_(0.0, 0.2)

    def forward(self, feats, coords, shape):
        x = self.input_proj(feats)
        shape = torch.Size([*shape[:4], x.shape[-1]])
        L = len(self.chans)
        conv_caches, down_caches, skips = [None] * L, [None] * (L - 1), [None] * (L - 1)
        for i in range(L):
            x, conv_caches[i] = self.down[i](x, coords, shape, conv_caches[i])
            if i < L - 1:
                skips[i] = (x, coords, shape)
                osh = torch.Size([shape[0]] + [-(-int(s) // 2) for s in shape[1:4]] + [shape[4]])
                x, coords, shape, down_caches[i] = self.pool[i](x, coords, shape, output_shape=osh)
                x = self.pool_lin[i](x)
                shape = torch.Size([*shape[:4], x.shape[-1]])
        x, conv_caches[L - 1] = self.bottleneck(x, coords, shape, conv_caches[L - 1])
        for i in reversed(range(L - 1)):
            sx, sc, ss = skips[i]
            x = self.up_lin[i](x)
            shape = torch.Size([*shape[:4], x.shape[-1]])
            x, coords, shape, _ = self.up[i](x, coords, shape, output_coords=sc, output_shape=ss,
                                             neighbor_cache=down_caches[i].T)
            x = x + sx
            x, conv_caches[i] = self.up_blocks[i](x, coords, shape, conv_caches[i])
        return self.out_proj(x), conv_caches, down_caches


def _np(p):
    return p.detach().double().cpu().numpy()


def _ref_forward(m: UNet, feats, coords, shape):
    """fp64 restatement with the oracle's sparse operators."""
    def lin(l, x):
        return x @ _np(l.weight).T + _np(l.bias)

    def block(b, x, nm):
        mu = x.mean(1, keepdims=True)
        var = ((x - mu) ** 2).mean(1, keepdims=True)
        h = (x - mu) / np.sqrt(var + 1e-6) * _np(b.norm1.weight) + _np(b.norm1.bias)
        h = h / (1.0 + np.exp(-h))
        h = ocv.conv_float(h, nm, _np(b.conv1.weight), _np(b.conv1.bias), dtype=np.float64)
        h = h / (1.0 + np.exp(-h))
        h = ocv.conv_float(h, nm, _np(b.conv2.weight), _np(b.conv2.bias), dtype=np.float64)
        return h + x

    L = len(m.chans)
    x = lin(m.input_proj, feats.astype(np.float64))
    c, shp = coords, tuple(shape[:4])
    maps, parents, skips = [], [], []
    for i in range(L):
        maps.append(ost.nmap_sorted(c, shp))
        x = block(m.down[i], x, maps[i])
        if i < L - 1:
            skips.append(x)
            osh = (shp[0],) + tuple(-(-s // 2) for s in shp[1:])
            oc, parent, _, _ = opl.pool_cache(c, shp, (2, 2, 2), osh)
            parents.append(parent)
            x = lin(m.pool_lin[i], opl.sparse_pool(x, parent, len(oc)).astype(np.float64))
            c, shp = oc, osh
    x = block(m.bottleneck, x, maps[L - 1])
    for i in reversed(range(L - 1)):
        x = opl.sparse_upsample(lin(m.up_lin[i], x), parents[i]) + skips[i]
        x = block(m.up_blocks[i], x, maps[i])
    return lin(m.out_proj, x), maps, parents


def test_multilevel_unet_through_the_shim(gpu):
    announce("3-level sparse U-Net through flex_gemm (conv, pool, upsample)")
    torch.manual_seed(0)
    cfg = spec.StepConfig("u", 48, 64, 50.0, 50.0, 32.0, 24.0, 16, 1, "int8", seed=11)
    sc = spec.make_scene(cfg)
    pts = np.stack([sc.points, sc.points * np.float32(1.02)])
    _, coords, Z, _ = ost.voxelize(pts)
    coords = coords.astype(np.int32)
    shape = (2, cfg.H, cfg.W, Z)
    feats = pts.reshape(-1, 3).astype(np.float32)
    m = UNet().to(gpu)
    with torch.no_grad():
        out, conv_caches, down_caches = m(torch.from_numpy(feats).to(gpu), torch.from_numpy(coords).to(gpu),
                                          torch.Size([*shape, 3]))
    torch.cuda.synchronize()
    ref, maps, parents = _ref_forward(m, feats, coords, shape)
    got = out.double().cpu().numpy()
    assert got.shape == ref.shape == (coords.shape[0], 1)
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(ref).max()
    # the caches the shim built are the reference's structures
    for i, cc in enumerate(conv_caches):
        assert np.array_equal(cc.nmap.cpu().numpy(), maps[i])
    for i, dc in enumerate(down_caches):
        assert np.array_equal(dc.parent.cpu().numpy(), parents[i])
