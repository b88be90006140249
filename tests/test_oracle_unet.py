"""The oracle's refiner composition against the reference's own modules, and the multi-level int8 arithmetic.

tests/golden/refiner_vectors.npz holds vectors that tests/golden/make_refiner_vectors.py recorded from the
reference's SparseResBlock3d, Sparse3DUNet and enable_refiner_qat (run over its bundled CPU flex_gemm): the block,
the level structure, every stage of a 3-level U-Net with encoder conditioning, prompt features and encoder bias map,
in fp32 and quantisation-aware. oracle/blocks.py and oracle/unet.py must reproduce them to fp32 rounding: the tests
allow 2e-6 of the stage's largest magnitude (a wrong block order, skip, pool/upsample order, concatenation order or
quantiser placement moves values by O(1)).
"""
import dataclasses

import numpy as np
import pytest

from oracle import blocks as ob
from oracle import structure as ost
from oracle import unet as ou
from oracle.numerics import quant_i8
from promptmoge_amd import spec
from promptmoge_amd import unet_weights as uw
from promptmoge_amd.spec import BlockW

GOLDEN = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "refiner_vectors.npz")
STAGES = ("down0", "pool0", "down1", "pool1", "down2", "enc_lin", "fuse", "bott", "dec0", "dec1")


def _close(got, ref, rel=2e-6):
    scale = max(float(np.abs(ref).max()), 1e-30)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    assert err <= rel * scale, (err, scale)


def _golden_unet():
    g = GOLDEN
    sd = {k[len("unet.sd."):]: g[k] for k in g.files if k.startswith("unet.sd.")}
    clips = {k[len("unet.clip."):]: float(g[k]) for k in g.files if k.startswith("unet.clip.")}
    w = uw.unet_from_state_dict(sd, factors=[2, 2], clips=clips)
    c = g["unet.coords"]
    shape = tuple(int(v) for v in g["unet.shape"][:4])
    levels = ou.build_levels(c, shape, w.factors, zkeys=c[:, 3].reshape(shape[:3]))
    return w, levels, sd, clips


def test_block_matches_reference():
    g = GOLDEN
    sd = {k[len("block.sd."):]: g[k] for k in g.files if k.startswith("block.sd.")}
    blk = BlockW(sd["norm1.weight"], sd["norm1.bias"], sd["conv1.weight"], sd["conv1.bias"], sd["conv2.weight"],
                 sd["conv2.bias"])
    c = g["block.coords"]
    B, H, W = (int(v) for v in g["block.shape"][:3])
    nmap = ost.nmap_column(c[:, 3].reshape(B, H, W))
    _close(ob.resblock(g["block.feats"], nmap, blk, "fp32"), g["block.out"])
    # a plausible misreading fails: the skip taken after the second SiLU, or the block without its skip
    h = ob.silu(ob.layer_norm(g["block.feats"], blk.gamma, blk.beta))
    no_skip = ob.conv_float(ob.silu(ob.conv_float(h, nmap, blk.w1, blk.b1)), nmap, blk.w2, blk.b2)
    with pytest.raises(AssertionError):
        _close(no_skip, g["block.out"])


def test_unet_levels_match_reference():
    w, levels, _, _ = _golden_unet()
    assert [lv.M for lv in levels][0] == GOLDEN["unet.coords"].shape[0]
    for k in (1, 2):
        assert np.array_equal(levels[k].coords, GOLDEN[f"unet.fp32.level{k}.coords"])
    assert len({tuple(r) for r in levels[1].coords[:, :3]}) < levels[1].M  # some columns hold several voxels


@pytest.mark.parametrize("mode,key", [("fp32", "fp32"), ("fakequant", "qat")])
def test_unet_stages_match_reference(mode, key):
    w, levels, _, _ = _golden_unet()
    g = GOLDEN
    tr = {}
    out = ou.forward(g["unet.feats"], levels, w, g["unet.enc"], g["unet.prompt"], g["unet.bias"], mode=mode,
                     trace=tr)
    for st in STAGES:
        _close(tr[st], g[f"unet.{key}.{st}"])
    _close(out, g[f"unet.out_{key}"][:, 0])


def test_unet_without_bias_map_or_prompt_differs():
    """The encoder bias map and the prompt features enter the result (the comparison above is not blind to them)."""
    w, levels, _, _ = _golden_unet()
    g = GOLDEN
    ref = g["unet.out_fp32"][:, 0]
    for args in [(g["unet.prompt"], None), (None, g["unet.bias"])]:
        out = ou.forward(g["unet.feats"], levels, w, g["unet.enc"], *args, mode="fp32")
        assert np.abs(out - ref).max() > 1e-3


def test_state_dict_reader_takes_qat_names():
    """A QAT checkpoint stores masters under .parametrizations.weight.original and clips as aq_<path>.clip
    (qat.py:111-115): the reader gives the same refiner as from the plain names plus clips."""
    w, _, sd, clips = _golden_unet()
    qsd = {}
    for k, v in sd.items():
        mod, _, leaf = k.rpartition(".")
        quantised = any(mod == p or mod.startswith(p + ".") for p in clips) and leaf == "weight"
        qsd[f"{mod}.parametrizations.weight.original" if quantised else k] = v
    for p, c in clips.items():
        qsd["aq_" + p.replace(".", "_") + ".clip"] = np.array(c, np.float32)
    w2 = uw.unet_from_state_dict(qsd, factors=[2, 2])
    assert w2.channels == w.channels == [8, 16, 16] and w2.enc_channels == 24
    for path, a in w.quantised_layers().items():
        b = w2.quantised_layers()[path]
        if hasattr(a, "clip1"):
            assert np.array_equal(a.w1, b.w1) and np.float32(a.clip1) == np.float32(b.clip1)
        else:
            assert np.array_equal(a.w, b.w) and np.float32(a.clip) == np.float32(b.clip)
    assert [len(s) for s in w2.down] == [1, 2, 1] and [len(s) for s in w2.dec] == [2, 1] and len(w2.bott) == 1


# ------------------------------------------------------------------------------------------------ int8 arithmetic
def _synthetic(channels=(16, 32, 32), seed=3, B=2, H=16, W=24, enc_c=32):
    w = uw.make_unet_weights(list(channels), enc_c, enc_blocks=[1, 2, 1], dec_blocks=[2, 1], factors=[2, 2],
                             seed=seed)
    cfg = spec.StepConfig("u", H, W, 0.9 * W, 0.9 * W, W / 2, H / 2, channels[0], 1, "int8", seed=seed)
    pts = np.stack([spec.make_scene(cfg, seed=seed + 7 * b).points for b in range(B)])
    rng = np.random.default_rng(seed)
    enc = rng.normal(0, 1, (B, enc_c, H // 4, W // 4)).astype(np.float32)
    bias = rng.normal(0, 0.1, (B, channels[-1], H // 4, W // 4)).astype(np.float32)
    M = B * H * W
    pf = np.stack([rng.normal(0, 0.05, M), rng.uniform(0, 1, M)], 1).astype(np.float32)
    zq, coords, zext, _ = ost.voxelize(pts)
    levels = ou.build_levels(coords, (B, H, W, zext), w.factors, zkeys=zq)
    w = ou.calibrate(w, levels, pts.reshape(M, 3), enc, pf, bias)
    return w, levels, pts.reshape(M, 3), enc, pf, bias


def test_state_dict_without_clips_is_refused():
    """A plain state dict carries no aq_*.clip entries; without `clips` the reader refuses it and names the first
    quantised layer it meets, instead of assuming a clip (which would saturate that layer's int8 input)."""
    _, _, sd, clips = _golden_unet()
    with pytest.raises(ValueError, match="activation clip"):
        uw.unet_from_state_dict(sd, factors=[2, 2])
    partial = dict(clips)
    missing = sorted(partial)[0]
    del partial[missing]
    with pytest.raises(ValueError, match=missing.replace(".", r"\.")):
        uw.unet_from_state_dict(sd, factors=[2, 2], clips=partial)


def test_int8_unet_matches_fakequant_statistically():
    """The deployed int8 arithmetic and the QAT fake-quant formulation evaluate one quantised model in different
    fp32 orders: a value within an ulp of a rounding tie may take the neighbouring code and propagate. Median error
    at fp32 rounding, mean < 1e-4 of the output scale, at most 1 % of voxels beyond 1e-3 of it."""
    w, levels, feats, enc, pf, bias = _synthetic()
    o8 = ou.forward(feats, levels, w, enc, pf, bias, mode="int8")
    oq = ou.forward(feats, levels, w, enc, pf, bias, mode="fakequant")
    of = ou.forward(feats, levels, w, enc, pf, bias, mode="fp32")
    scale = float(np.abs(oq).max())
    d = np.abs(o8.astype(np.float64) - oq) / scale
    assert np.median(d) < 1e-6 and d.mean() < 1e-4 and (d > 1e-3).mean() < 0.01, (np.median(d), d.mean())
    assert np.abs(of - oq).max() > 10 * np.abs(o8 - oq).max()  # quantisation matters more than the order


def test_metal_requant_differs_from_qat_only_at_ties():
    """The deployed requantisation rint(x * (127/clip)) and the QAT rule round(x / (clip/127)) (qat.py:36) give the
    same code except where x * 127 / clip lies within a few ulps of a half-integer. Checked on random values, on
    values built next to ties, and on every quantised layer's input of an int8 U-Net."""
    rng = np.random.default_rng(0)
    clips = rng.uniform(0.05, 20, 64).astype(np.float32)
    xs = [rng.uniform(-1.2, 1.2, 200_000).astype(np.float32) * c for c in clips[:8]]
    ties = (rng.integers(-130, 130, 200_000) + 0.5).astype(np.float64)
    near = [(ties * (float(c) / 127.0) * (1 + rng.uniform(-4e-7, 4e-7, ties.size))).astype(np.float32)
            for c in clips[8:16]]
    w, levels, feats, enc, pf, bias = _synthetic()
    rec = {}
    ou.forward(feats, levels, w, enc, pf, bias, mode="fp32", record=rec)
    layers = w.quantised_layers()
    acts = []
    for path, layer in layers.items():
        if hasattr(layer, "clip1"):
            acts += [(rec[path + ".conv1"], layer.clip1), (rec[path + ".conv2"], layer.clip2)]
        else:
            acts.append((rec[path], layer.clip))
    cases = list(zip(xs, clips[:8])) + list(zip(near, clips[8:16])) + acts
    flips = 0
    for x, clip in cases:
        a = quant_i8(x, ob.act_mult(clip)).astype(np.int32)
        b = ob.qat_codes(x, clip).astype(np.int32)
        diff = a != b
        flips += int(diff.sum())
        if diff.any():
            t = x[diff].astype(np.float64) * 127.0 / float(np.float32(clip))
            frac = np.abs(t - np.floor(t) - 0.5)
            assert (frac <= 8 * np.spacing(np.abs(t).astype(np.float32)).astype(np.float64)).all()
            assert (np.abs(a[diff] - b[diff]) == 1).all()
    assert flips > 0  # the near-tie values do exercise the difference


def test_refiner_bin_round_trip(tmp_path):
    """save_refiner_bin writes export/refiner.py's layout; load_refiner_bin reads it back: the same int8 weights
    and scales (kept as stored), clips, fp16 biases and projections, and the same int8 forward."""
    w, levels, feats, enc, pf, bias = _synthetic(enc_c=32)
    w1 = uw.fp16_exact(dataclasses.replace(
        w, down=[st[:1] for st in w.down], dec=[st[:1] for st in w.dec]))
    uw.save_refiner_bin(w1, tmp_path, 16, 24, uv_bias=np.zeros((32, 4, 6), np.float32))
    w2, man, uv = uw.load_refiner_bin(tmp_path)
    assert man["levels"] == 3 and man["channels"] == [16, 32, 32] and man["R"] == 4 and man["C"] == 6
    assert uv.shape == (32, 4, 6)
    for path, a in w1.quantised_layers().items():
        b = w2.quantised_layers()[path]
        pairs = [(a.w1, b.w1), (a.w2, b.w2)] if hasattr(a, "w1") else [(a.w, b.w)]
        for x, y in pairs:
            qa, sa = uw.quantized(x)
            qb, sb = uw.quantized(y)
            assert np.array_equal(qa, qb) and np.array_equal(sa, sb)
    o1 = ou.forward(feats, levels, w1, enc, pf, bias, mode="int8")
    o2 = ou.forward(feats, levels, w2, enc, pf, bias, mode="int8")
    assert np.array_equal(o1, o2)


def test_unet_refiner_refuses_widths_beyond_256():
    """The int8 U-Net runs widths up to 256 (the deployed 32 64 128 256 256 refiners, train.py:124); the stock
    512-wide refiner is refused when the module is built, before any device work."""
    from promptmoge_amd.unet import UNetRefiner

    w = uw.make_unet_weights([16, 32, 512], 32, seed=0)
    with pytest.raises(ValueError, match="level widths"):
        UNetRefiner(w)


def test_teacher_state_dict_needs_no_clips():
    """The fp16 teacher quantises nothing: its plain state dict loads without clips (they are left NaN; the
    reference module's own golden state dict, whose 8-wide level 0 the device does not take, so the reader is
    called directly), and the int8 reader still refuses the same dict."""
    _, _, sd, _ = _golden_unet()
    w = uw.unet_from_state_dict(sd, factors=[2, 2], require_clips=False)
    assert w.channels == [8, 16, 16] and np.isnan(w.enc.clip) and np.isnan(w.down[0][0].clip1)
    with pytest.raises(ValueError, match="activation clip"):
        uw.unet_from_state_dict(sd, factors=[2, 2])
