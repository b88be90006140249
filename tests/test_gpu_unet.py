"""GPU parity of the multi-level int8 refiner (UNetRefiner, csrc/pmg_unet.hip) against oracle/unet.py.

Bit for bit on identical seeded inputs: every level's voxel count, coordinates, parents and submanifold map (tap
masks too), the stream after every stage, the encoder tokens and the (M, 1) output; the forward with keys from the
log depth (coords None) equals the one with _voxelize's coords; graph replays repeat the first result. The oracle's
composition is pinned against the reference's own Sparse3DUNet (tests/test_oracle_unet.py).
"""
import numpy as np
import pytest
import torch

from oracle import structure as ost
from oracle import unet as ou
from promptmoge_amd import spec
from promptmoge_amd import unet_weights as uw
from promptmoge_amd.unet import UNetRefiner

from conftest import announce

pytestmark = pytest.mark.gpu

CASES = {
    # name: (channels, enc_blocks, dec_blocks, bottleneck, B, H, W, enc_channels, seed)
    "small3": ([16, 32, 32], [1, 2, 1], [2, 1], 1, 2, 32, 48, 32, 3),
    "wide4": ([32, 64, 128, 256], [1, 1, 1, 1], [1, 1, 1], 1, 1, 64, 96, 64, 5),
    "modelB5": ([32, 64, 128, 256, 256], [1, 1, 1, 1, 1], [1, 1, 1, 1], 1, 1, 240, 320, 1024, 7),
    # the widths that take the generic spconv_k and rows_ln_k<48 / 96 / 192> at levels >= 1
    "odd3": ([48, 96, 192], [1, 1, 1], [1, 1], 1, 1, 48, 64, 48, 13),
}


def _setup(name):
    channels, eb, db, bb, B, H, W, enc_c, seed = CASES[name]
    L = len(channels)
    ds = 2 ** (L - 1)
    w = uw.make_unet_weights(channels, enc_c, enc_blocks=eb, dec_blocks=db, bottleneck_blocks=bb, seed=seed)
    cfg = spec.StepConfig("u", H, W, 0.9 * W, 0.9 * W, W / 2, H / 2, channels[0], 1, "int8", seed=seed)
    pts = np.stack([spec.make_scene(cfg, seed=seed + 11 * b).points for b in range(B)])
    rng = np.random.default_rng(seed)
    enc = rng.normal(0, 1, (B, enc_c, H // ds, W // ds)).astype(np.float32)
    bias = rng.normal(0, 0.1, (B, channels[-1], H // ds, W // ds)).astype(np.float32)
    M = B * H * W
    pf = np.stack([rng.normal(0, 0.05, M), rng.uniform(0, 1, M)], 1).astype(np.float32)
    zq, coords, zext, _ = ost.voxelize(pts)
    levels = ou.build_levels(coords, (B, H, W, zext), w.factors, zkeys=zq)
    w = ou.calibrate(w, levels, pts.reshape(M, 3), enc, pf, bias)
    return w, levels, pts, coords, enc, bias, pf, (B, H, W, zext)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("name", list(CASES))
def test_unet_int8_matches_oracle(gpu, name):
    announce(f"unet int8 forward case={name}")
    w, levels, pts, coords, enc, bias, pf, (B, H, W, Z) = _setup(name)
    M = B * H * W
    L = w.levels
    mod = UNetRefiner(w)
    shape = torch.Size([B, H, W, Z, 3])
    tf, tc, te, tb, tp = (_t(a, gpu) for a in (pts.reshape(M, 3), coords, enc, bias, pf))
    out = mod(tf, tc, shape, te, prompt_feats=tp, encoder_bias_map=tb)
    torch.cuda.synchronize()
    bufs = {}
    counts = mod.buffer("counts", 0).cpu().numpy()
    for k in range(L):
        Mk = int(counts[k])
        bufs[k] = {"coords": mod.buffer("coords", k).cpu().numpy()[:Mk], "down": mod.buffer("down", k).cpu().numpy()[:Mk],
                   "up": mod.buffer("up", k).cpu().numpy()[:Mk]}
        if k + 1 < L:
            bufs[k]["parent"] = mod.buffer("parent", k).cpu().numpy()[:Mk]
        if k > 0:
            bufs[k]["nmap"] = mod.buffer("nmap", k).cpu().numpy()[:, :Mk]
            bufs[k]["tile_mask"] = mod.buffer("tile_mask", k).cpu().numpy()[:(Mk + 15) // 16]
    enc_tok = mod.buffer("enc_tokens", 0).cpu().numpy()
    trace = {}
    ref = ou.forward(pts.reshape(M, 3), levels, w, enc, pf, bias, mode="int8", trace=trace)
    # structure
    assert [int(c) for c in counts] == [lv.M for lv in levels], (counts, [lv.M for lv in levels])
    for k in range(1, L):
        assert np.array_equal(bufs[k]["coords"], levels[k].coords), k
        assert np.array_equal(bufs[k]["nmap"].T, levels[k].nmap), k
        assert np.array_equal(bufs[k]["tile_mask"].view(np.uint32), ost.tile_masks(levels[k].nmap)), k
    for k in range(L - 1):
        assert np.array_equal(bufs[k]["parent"], levels[k + 1].parent), k
    # streams after every stage
    for k in range(L):
        assert np.array_equal(bufs[k]["down"], trace[f"down{k}"]), f"down{k}"
    assert np.array_equal(bufs[L - 1]["up"], trace["bott"])
    for i in range(L - 2):
        assert np.array_equal(bufs[L - 2 - i]["up"], trace[f"dec{i}"]), f"dec{i}"
    # level 0: the last convolution applies out_proj without storing the stream, which holds what enters the
    # last block
    last = trace[f"dec{L - 2}_blocks"]
    assert np.array_equal(bufs[0]["up"], last[-2]["x"] if len(last) > 1 else trace[f"dec{L - 2}_in"])
    top = levels[L - 1].coords.astype(np.int64)
    R, Cc = H >> (L - 1), W >> (L - 1)
    assert np.array_equal(enc_tok[(top[:, 0] * R + top[:, 1]) * Cc + top[:, 2]], trace["enc"])
    assert np.array_equal(out.cpu().numpy()[:, 0], ref)
    # the refiner moved something: its output is not a constant
    assert np.std(ref) > 1e-3


def test_unet_keys_from_depth_and_graph_replay(gpu):
    """coords None: the level-0 keys come from rint(logz * 256) - per-batch min (_voxelize, v3.py:332-340) on the
    device, giving the same structure and output; a graph replay repeats it; without the prompt and the bias map the
    output matches the oracle run without them."""
    announce("unet keys from depth, replay, no prompt / bias map")
    w, levels, pts, coords, enc, bias, pf, (B, H, W, Z) = _setup("small3")
    M = B * H * W
    mod = UNetRefiner(w)
    shape = torch.Size([B, H, W, Z, 3])
    tf, tc, te, tb, tp = (_t(a, gpu) for a in (pts.reshape(M, 3), coords, enc, bias, pf))
    a = mod(tf, tc, shape, te, prompt_feats=tp, encoder_bias_map=tb)
    b = mod(tf, None, shape, te, prompt_feats=tp, encoder_bias_map=tb)
    c = mod(tf, tc, shape, te, prompt_feats=tp, encoder_bias_map=tb)
    d = mod(tf, tc, shape, te)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert np.array_equal(a.cpu().numpy(), c.cpu().numpy())
    # level 0's coordinates live at one address whichever graph ran last: a replay of the given-coordinates graph
    # after the from-depth one exposes the coordinates it was given
    tc2 = tc.clone()
    tc2[:, 3] += 1
    mod(tf, tc2, shape, te, prompt_feats=tp, encoder_bias_map=tb)
    torch.cuda.synchronize()
    assert np.array_equal(mod.buffer("coords", 0).cpu().numpy()[:M], tc2.cpu().numpy())
    ref_d = ou.forward(pts.reshape(M, 3), levels, w, enc, None, None, mode="int8")
    assert np.array_equal(d.cpu().numpy()[:, 0], ref_d)
    assert np.abs(a.cpu().numpy() - d.cpu().numpy()).max() > 1e-4


def test_unet_reused_inputs_read_in_place(gpu):
    """Inputs passed again (the same tensors as the previous call) are read in place by their own captured graph:
    the result equals the staged call's, and a change written into those tensors in place is seen by the next
    replay (the graph reads the buffers at replay time)."""
    announce("unet reused input tensors read in place")
    w, levels, pts, coords, enc, bias, pf, (B, H, W, Z) = _setup("small3")
    M = B * H * W
    mod = UNetRefiner(w)
    shape = torch.Size([B, H, W, Z, 3])
    tf, tc, te, tb, tp = (_t(a, gpu) for a in (pts.reshape(M, 3), coords, enc, bias, pf))
    first = mod(tf, tc, shape, te, prompt_feats=tp, encoder_bias_map=tb)  # staged
    again = [mod(tf, tc, shape, te, prompt_feats=tp, encoder_bias_map=tb) for _ in range(3)]  # in place
    te.mul_(0.5)
    tp[:, 0] += 0.01
    changed = mod(tf, tc, shape, te, prompt_feats=tp, encoder_bias_map=tb)
    staged = mod(tf.clone(), tc, shape, te.clone(), prompt_feats=tp.clone(), encoder_bias_map=tb)
    torch.cuda.synchronize()
    for o in again:
        assert np.array_equal(first.cpu().numpy(), o.cpu().numpy())
    assert np.array_equal(changed.cpu().numpy(), staged.cpu().numpy())
    ref = ou.forward(pts.reshape(M, 3), levels, w, te.cpu().numpy(), tp.cpu().numpy(), bias, mode="int8")
    assert np.array_equal(changed.cpu().numpy()[:, 0], ref)
    assert np.abs(changed.cpu().numpy() - first.cpu().numpy()).max() > 1e-4


def test_unet_from_refiner_bin(gpu, tmp_path):
    """A refiner exported in the Metal engine's format (refiner.bin / refiner.json) and loaded back: the GPU module
    built from the file equals the oracle on the loaded (stored int8) weights, with the file's uv_bias as the bias
    map."""
    announce("unet from refiner.bin")
    w, levels, pts, coords, enc, bias, pf, (B, H, W, Z) = _setup("small3")
    w1 = uw.fp16_exact(uw.UNetW(**{**w.__dict__, "down": [st[:1] for st in w.down], "dec": [st[:1] for st in w.dec]}))
    uv = np.random.default_rng(9).normal(0, 0.1, (w.channels[-1], H // 4, W // 4)).astype(np.float32)
    uw.save_refiner_bin(w1, tmp_path, H, W, uv_bias=uv)
    mod, uv2 = UNetRefiner.from_refiner_bin(tmp_path)
    assert np.array_equal(uv, uv2)
    w2 = mod.host_weights
    M = B * H * W
    bmap = np.broadcast_to(uv2[None], (B,) + uv2.shape).copy()
    out = mod(_t(pts.reshape(M, 3), gpu), _t(coords, gpu), torch.Size([B, H, W, Z, 3]), _t(enc, gpu),
              prompt_feats=_t(pf, gpu), encoder_bias_map=_t(bmap, gpu))
    ref = ou.forward(pts.reshape(M, 3), levels, w2, enc, pf, bmap, mode="int8")
    assert np.array_equal(out.cpu().numpy()[:, 0], ref)


# ---- the fp16 teacher (PromptMoGe-L): oracle/blocks.py "fp16" arithmetic ------------------------------------------
F16_CASES = {
    # name: (channels, enc_blocks, dec_blocks, bottleneck, B, H, W, enc_channels, seed)
    "teacher5_small": ([32, 64, 128, 256, 512], [1, 1, 1, 1, 1], [1, 1, 1, 1], 1, 1, 64, 96, 64, 5),
    "teacher5_240x320": ([32, 64, 128, 256, 512], [1, 1, 1, 1, 1], [1, 1, 1, 1], 1, 1, 240, 320, 256, 5),
    "f16_3lv_b2": ([16, 32, 64], [1, 2, 1], [2, 1], 1, 2, 32, 48, 32, 3),
}


def _rms(a):
    return float(np.sqrt(np.mean(np.square(np.asarray(a, np.float64)))))


@pytest.mark.parametrize("name", list(F16_CASES))
def test_unet_fp16_matches_oracle(gpu, name):
    """The stock 512-wide teacher U-Net (train.py:124) natively in fp16, against oracle/unet.py's "fp16" arithmetic
    (fp16 activations and weights in every conv and linear, fp32 accumulation, fp32 streams). The level structure is
    bit for bit. The values cannot be: the device sums in its MFMA order, and a different fp32 summation order moves
    fp16 roundings by one ulp, which the next LayerNorm and the wide coarse layers amplify (on these weights the
    oracle summed in fp32 instead of fp64 lands 1e-3 RMS away from itself at the output). So:
      * level 0's stream, before much amplification, within 1e-5 RMS of the oracle -- a tenth of what rounding to
        fp16 changes there (the fp32 module) -- so the device computes the teacher's fp16 arithmetic;
      * every level's stream and the (M, 1) output within three times that summation-order spread (RMS) of the
        oracle, and four times it at the worst element: the device differs from the oracle in two independent ways
        of that size -- its summation order, and its SiLU (hardware exp2 / reciprocal, within one fp16 ulp of the
        oracle's before the rounding) -- where the fp32-summed oracle differs in one."""
    announce(f"unet fp16 forward case={name}")
    channels, eb, db, bb, B, H, W, enc_c, seed = F16_CASES[name]
    L = len(channels)
    ds = 2 ** (L - 1)
    w = uw.make_unet_weights(channels, enc_c, enc_blocks=eb, dec_blocks=db, bottleneck_blocks=bb, seed=seed)
    cfg = spec.StepConfig("u", H, W, 0.9 * W, 0.9 * W, W / 2, H / 2, channels[0], 1, "int8", seed=seed)
    pts = np.stack([spec.make_scene(cfg, seed=seed + 11 * b).points for b in range(B)])
    rng = np.random.default_rng(seed)
    enc = rng.normal(0, 1, (B, enc_c, H // ds, W // ds)).astype(np.float32)
    bias = rng.normal(0, 0.1, (B, channels[-1], H // ds, W // ds)).astype(np.float32)
    M = B * H * W
    pf = np.stack([rng.normal(0, 0.05, M), rng.uniform(0, 1, M)], 1).astype(np.float32)
    zq, coords, zext, _ = ost.voxelize(pts)
    levels = ou.build_levels(coords, (B, H, W, zext), w.factors, zkeys=zq)
    mod = UNetRefiner(w, precision="fp16")
    shape = torch.Size([B, H, W, zext, 3])
    tf, tc, te, tb, tp = (_t(a, gpu) for a in (pts.reshape(M, 3), coords, enc, bias, pf))
    out = mod(tf, tc, shape, te, prompt_feats=tp, encoder_bias_map=tb)
    out2 = mod(tf, None, shape, te, prompt_feats=tp, encoder_bias_map=tb)  # keys from the depth, another graph
    torch.cuda.synchronize()
    counts = mod.buffer("counts", 0).cpu().numpy()
    assert [int(c) for c in counts] == [lv.M for lv in levels]
    for k in range(1, L):
        assert np.array_equal(mod.buffer("coords", k).cpu().numpy()[:levels[k].M], levels[k].coords), k
    assert np.array_equal(out.cpu().numpy(), out2.cpu().numpy())
    tr, tr_alt, tr32 = {}, {}, {}
    ref = ou.forward(pts.reshape(M, 3), levels, w, enc, pf, bias, mode="fp16", trace=tr)
    alt = ou.forward(pts.reshape(M, 3), levels, w, enc, pf, bias, mode="fp16", trace=tr_alt, acc=np.float32)
    ou.forward(pts.reshape(M, 3), levels, w, enc, pf, bias, mode="fp32", trace=tr32)
    d0 = mod.buffer("down", 0).cpu().numpy()[:M]
    r0 = tr["down0"]
    assert _rms(d0 - r0) <= 1e-5 * _rms(r0) and _rms(d0 - r0) <= 0.1 * _rms(tr32["down0"] - r0), (
        _rms(d0 - r0) / _rms(r0), _rms(tr32["down0"] - r0) / _rms(r0))
    pairs = [(mod.buffer("down", k).cpu().numpy()[:levels[k].M], tr[f"down{k}"], tr_alt[f"down{k}"], f"down{k}")
             for k in range(L)]
    pairs.append((out.cpu().numpy()[:, 0], ref, alt, "out"))
    for got, r, a, what in pairs:
        spread, spread_max = _rms(a - r), float(np.abs(a - r).max())
        err, err_max = _rms(got - r), float(np.abs(got - r).max())
        assert err <= 3 * spread + 1e-6 * _rms(r) and err_max <= 4 * spread_max + 1e-6 * float(np.abs(r).max()), (
            what, err / _rms(r), spread / _rms(r), err_max, spread_max)
