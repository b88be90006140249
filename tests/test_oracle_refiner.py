"""The oracle's deployed-arithmetic step (int8 codes, exact int32 accumulation, fp32 epilogues; fp16 teacher)
against the reference's own formulations of the same model: the fp32 fake-quant QAT path for int8 and the fp32
_fallback path for fp16.

fp16: depth within 1e-3 relative everywhere.
int8: the two formulations evaluate the same quantised model in different fp32 operation orders, so a value that
lands within an ulp of a rounding tie can take the neighbouring int8 code, and that one-step change propagates
through the later blocks (on a small map a single flip reaches a few percent of the voxels). The criterion is
therefore statistical: the median voxel agrees to fp32 rounding (1e-6), the mean relative depth error is < 1e-4,
and at most 0.5 % of voxels differ by more than 1e-3. (The GPU is compared
with the oracle's own order, op for op, and must match it bit for bit.)"""
import dataclasses

import numpy as np
import pytest

from oracle import refiner as rf
from oracle.blocks import resblock
from promptmoge_amd import spec


def _small(prec, C, seed):
    cfg = spec.StepConfig("s", 72, 96, 80.0, 80.0, 48.0, 36.0, C, 2, prec, seed=seed)
    sc = spec.make_scene(cfg)
    w = spec.calibrate(spec.make_weights(C, 2, seed=seed, precision=prec), sc, crop=64)
    return sc, w


@pytest.mark.parametrize("seed", [0, 1])
def test_int8_step_matches_fakequant_reference(seed):
    sc, w = _small("int8", 16, seed)
    pts, st, _ = rf.step(sc.points[None], sc.lidar[None], sc.conf[None], w, precision="int8", iters=10)
    ref = rf.step_fakequant(sc.points[None], sc.lidar[None], sc.conf[None], w, iters=10)
    d, dr = np.exp(pts[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
    rel = np.abs(d - dr) / dr
    assert np.median(rel) < 1e-6 and rel.mean() < 1e-4 and (rel > 1e-3).mean() < 5e-3, (rel.mean(), rel.max())
    # the refiner did move the depth, so the comparison is not vacuous
    assert np.abs(pts[..., 2] - sc.points[None, ..., 2]).mean() > 1e-3


def test_fp16_step_matches_fp32_reference():
    sc, w = _small("fp16", 16, 2)
    pts, _, _ = rf.step(sc.points[None], sc.lidar[None], sc.conf[None], w, precision="fp16", iters=10)
    # fp32 reference: the same model with fp32 operands everywhere (no activation rounding)
    w32 = dataclasses.replace(w, blocks=[dataclasses.replace(b) for b in w.blocks])
    B, H, W = 1, sc.points.shape[0], sc.points.shape[1]
    z, tg, m, d, c = rf.prompt_inputs(sc.points[None], sc.lidar[None], sc.conf[None])
    s, t = rf.fit_f64(z, tg, m, 10)
    r, g = rf.prompt_feats(sc.points[None], d, c, s, t)
    zq, _, _, _ = rf.voxelize(sc.points[None])
    nm = rf.nmap_column(zq)
    x = rf.input_proj(sc.points.reshape(-1, 3), w32, r.reshape(-1), g.reshape(-1))
    for blk in w32.blocks:  # the fp32 block, pinned against the reference's SparseResBlock3d (test_oracle_unet.py)
        x = resblock(x, nm, blk, "fp32")
    ref = sc.points[..., 2] + (x @ w32.out_w.reshape(-1) + w32.out_b[0]).reshape(H, W)
    rel = np.abs(np.exp(pts[0, ..., 2].astype(np.float64)) - np.exp(ref.astype(np.float64))) / np.exp(ref)
    assert rel.max() < 1e-3, rel.max()


def test_weights_from_reference_state_dict():
    """spec.weights_from_state_dict reads the reference module's parameter names (plain and QAT-parametrised)."""
    import torch
    from promptmoge_amd import spec

    w = spec.make_weights(32, 2, seed=3)
    sd = {"input_proj.weight": torch.from_numpy(w.in_w), "input_proj.bias": torch.from_numpy(w.in_b),
          "prompt_proj.weight": torch.from_numpy(w.pr_w), "prompt_proj.bias": torch.from_numpy(w.pr_b),
          "out_proj.parametrizations.weight.original": torch.from_numpy(w.out_w),
          "out_proj.bias": torch.from_numpy(w.out_b)}
    for k, b in enumerate(w.blocks):
        stage, idx = ("down_stages.0", k) if k == 0 else ("bottleneck_stage", k - 1)
        p = f"{stage}.{idx}"
        sd.update({f"{p}.norm1.weight": b.gamma, f"{p}.norm1.bias": b.beta,
                   f"{p}.conv1.parametrizations.weight.original": torch.from_numpy(b.w1), f"{p}.conv1.bias": b.b1,
                   f"{p}.conv2.weight": b.w2, f"{p}.conv2.bias": b.b2,
                   "aq_" + p.replace(".", "_") + "_conv1.clip": torch.tensor(b.clip1),
                   "aq_" + p.replace(".", "_") + "_conv2.clip": torch.tensor(b.clip2)})
    got = spec.weights_from_state_dict(sd)
    assert got.C == 32 and len(got.blocks) == 2
    for a, b in zip(got.blocks, w.blocks):
        for f in ("gamma", "beta", "w1", "b1", "w2", "b2"):
            assert np.array_equal(getattr(a, f), getattr(b, f)), f
        assert a.clip1 == pytest.approx(b.clip1) and a.clip2 == pytest.approx(b.clip2)
    assert np.array_equal(got.out_w, w.out_w) and np.array_equal(got.in_w, w.in_w)


def test_int8_refiner_refuses_missing_clips():
    """weights_from_state_dict leaves a clip it cannot find as NaN (the fp16 refiner never reads it); building the
    int8 device weights from it raises, naming the layer."""
    import torch
    from promptmoge_amd import spec
    from promptmoge_amd.refiner import DeviceWeights

    w = spec.make_weights(16, 2, seed=1)
    sd = {"input_proj.weight": w.in_w, "input_proj.bias": w.in_b, "out_proj.weight": w.out_w,
          "out_proj.bias": w.out_b}
    for k, b in enumerate(w.blocks):
        p = f"down_stages.0.{k}"
        sd.update({f"{p}.norm1.weight": b.gamma, f"{p}.norm1.bias": b.beta, f"{p}.conv1.weight": b.w1,
                   f"{p}.conv1.bias": b.b1, f"{p}.conv2.weight": b.w2, f"{p}.conv2.bias": b.b2})
    got = spec.weights_from_state_dict(sd, stages=("down_stages.0",))
    assert np.isnan(got.blocks[0].clip1)
    with pytest.raises(ValueError, match="block 0 conv1"):
        DeviceWeights(got, "int8", device="cpu")
    clips = {f"down_stages.0.{k}.conv{i}": 2.0 for k in range(2) for i in (1, 2)}
    ok = spec.weights_from_state_dict(sd, stages=("down_stages.0",), clips=clips)
    DeviceWeights(ok, "int8", device="cpu")
    DeviceWeights(got, "fp16", device="cpu")


# ---- output gate and elastic anchor (v3.py:565-573, 386-393) -------------------------------------------------
def test_lidar_uncertainty_closed_form():
    """u = 1 - c * (1 - clamp((d - 3) / 2, 0, 1)) where the LiDAR has a value, else 1 (prompt_stem.py:28-29)."""
    d = np.array([[[2.0, 4.0, 6.0, 3.0, 5.0, 4.0, 0.0, np.nan, np.inf, -1.0]]], np.float32)
    c = np.array([[[1.0, 1.0, 1.0, 1.0, 1.0, 0.5, 1.0, 1.0, 1.0, 1.0]]], np.float32)
    u = rf.lidar_uncertainty(d, c)
    np.testing.assert_array_equal(u[0, 0], np.float32([0.0, 0.5, 1.0, 0.0, 1.0, 0.75, 1.0, 1.0, 1.0, 1.0]))
    # no confidence: full uncertainty whatever the range
    assert np.all(rf.lidar_uncertainty(np.float32([[[1.0, 4.0, 9.0]]]), np.zeros((1, 1, 3), np.float32)) == 1.0)


def test_output_gate_limits():
    rng = np.random.default_rng(0)
    cur = rng.normal(0.5, 0.3, (1, 4, 5)).astype(np.float32)
    ref = (cur + rng.normal(0, 0.05, cur.shape)).astype(np.float32)
    d = np.full(cur.shape, 2.0, np.float32)  # inside the 3 m knee: u = 1 - c
    c1 = np.ones(cur.shape, np.float32)
    # floor 0 and a confident close pixel (u = 0): no update at all
    np.testing.assert_array_equal(rf.output_gate(cur, ref, d, c1, 0.0), cur)
    # floor 1: the full update (up to the rounding of cur + (ref - cur))
    np.testing.assert_allclose(rf.output_gate(cur, ref, d, c1, 1.0), ref, rtol=0, atol=1e-6)
    # u = 1 (no confidence): the full update for any floor
    np.testing.assert_allclose(rf.output_gate(cur, ref, d, np.zeros_like(c1), 0.1), ref, rtol=0, atol=1e-6)
    # half-way: floor 0, c = 1, d = 4 m -> u = 0.5 -> cur + 0.5 (ref - cur)
    out = rf.output_gate(cur, ref, np.full(cur.shape, 4.0, np.float32), c1, 0.0)
    np.testing.assert_allclose(out, 0.5 * (cur.astype(np.float64) + ref), rtol=0, atol=1e-6)


def test_anchor_pull_limits():
    rng = np.random.default_rng(1)
    logz = rng.normal(0.3, 0.2, (2, 3, 4)).astype(np.float32)
    d = rng.uniform(1.0, 4.0, logz.shape).astype(np.float32)
    c = np.ones(logz.shape, np.float32)
    s, t = np.float32([1.3, 0.8]), np.float32([0.05, -0.02])
    np.testing.assert_array_equal(rf.anchor_pull(logz, d, c, s, t, 0.0), logz)  # beta 0: off
    # beta 1, full confidence: the LiDAR in the affine frame, log((d - t) / s), computed here in fp64
    want = np.log((d.astype(np.float64) - t[:, None, None]) / s[:, None, None])
    np.testing.assert_allclose(rf.anchor_pull(logz, d, c, s, t, 1.0), want, rtol=0, atol=2e-6)
    # no LiDAR value or no confidence: the gate is 0
    d2 = d.copy()
    d2[0, 0, 0] = 0.0
    c2 = c.copy()
    c2[1, 2, 3] = 0.0
    out = rf.anchor_pull(logz, d2, c2, s, t, 0.7)
    assert out[0, 0, 0] == logz[0, 0, 0] and out[1, 2, 3] == logz[1, 2, 3]
    # half strength: half-way between logz and the target
    half = rf.anchor_pull(logz, d, c, s, t, 0.5)
    np.testing.assert_allclose(half, 0.5 * (logz + want), rtol=0, atol=2e-6)


# ------------------------------------------------------------------------------------------------ closed forms
def _level0(C=16, seed=5, n_blocks=2):
    cfg = spec.StepConfig("c", 24, 32, 30.0, 30.0, 16.0, 12.0, C, n_blocks, "int8", seed=seed)
    sc = spec.make_scene(cfg)
    w = spec.calibrate(spec.make_weights(C, n_blocks, seed=seed), sc, crop=32)
    zq, _, _, _ = rf.voxelize(sc.points[None])
    rng = np.random.default_rng(seed)
    M = cfg.H * cfg.W
    pf = np.stack([rng.normal(0, 0.05, M), rng.uniform(0, 1, M)], 1).astype(np.float32)
    return cfg, sc, w, zq, pf


def test_zero_conv2_blocks_are_the_identity():
    """Every conv2 weight and bias zero: each SparseResBlock3d returns its input (skip only, flex_sparse_blocks.py:
    75), so the module is out_proj(input_proj(f) + prompt_proj(pf)) (sparse_unet.py:189-192, 258), here checked
    against an independent float64 evaluation."""
    cfg, sc, w, zq, pf = _level0()
    w0 = dataclasses.replace(w, blocks=[dataclasses.replace(b, w2=np.zeros_like(b.w2), b2=np.zeros_like(b.b2))
                                        for b in w.blocks])
    f = sc.points.reshape(-1, 3)
    got = rf.forward(f, zq, cfg.H, cfg.W, w0, pf, precision="int8")
    f64 = lambda a: np.asarray(a, np.float64)
    x = f @ f64(w.in_w).T + f64(w.in_b) + pf @ f64(w.pr_w).T + f64(w.pr_b)
    ref = x @ f64(w.out_w).reshape(-1) + f64(w.out_b)[0]
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    # and the blocks do act when conv2 is not zero
    assert np.abs(rf.forward(f, zq, cfg.H, cfg.W, w, pf, precision="int8") - ref).max() > 1e-3


def test_constant_layernorm_and_centre_tap_conv1():
    """gamma = 0, beta = b: LayerNorm returns b in every row, so conv1's input codes are quant(silu(b), 127/clip1)
    in every row; with only the centre tap of conv1 non-zero (v = 13, the voxel itself, present in every row),
    acc1[m, n] = sum_c W[n, 13, c] * q[c] for every m."""
    cfg, sc, w, zq, pf = _level0(n_blocks=1)
    b = w.blocks[0]
    rng = np.random.default_rng(7)
    beta = rng.normal(0, 1.0, b.beta.shape).astype(np.float32)
    w1 = np.zeros_like(b.w1)
    w1[:, 1, 1, 1, :] = rng.normal(0, 0.05, (b.w1.shape[0], b.w1.shape[-1]))
    wc = dataclasses.replace(w, blocks=[dataclasses.replace(b, gamma=np.zeros_like(b.gamma), beta=beta, w1=w1)])
    trace = {}
    rf.step(sc.points[None], sc.lidar[None], sc.conf[None], wc, precision="int8", iters=4, trace=trace)
    blk = trace["blocks"][0]
    from oracle.numerics import silu_f32
    codes = np.clip(np.rint(silu_f32(beta) * (np.float32(127) / np.float32(b.clip1))), -127, 127).astype(np.int64)
    assert (blk["q1"] == codes[None, :]).all()
    q, _ = rf.quantize_weight(w1)
    expect = q.reshape(q.shape[0], 27, -1)[:, 13, :].astype(np.int64) @ codes
    assert (blk["acc1"] == expect[None, :]).all()


def test_prompt_features_hand_built():
    """_lidar_in_affine_frame's residual and gate (v3.py:371-383) and the channel order [residual, gate]
    (v3.py:552-554) on hand-built pixels, (s, t) = (2, 0.5): d_aff = (d - t) / max(s, 1e-6)."""
    logz = np.array([[0.3, -0.2, 0.1, 0.7, 0.05, 1.1]], np.float32)
    pts = np.zeros((1, 1, 6, 3), np.float32)
    pts[..., 2] = logz
    d = np.array([[[2.5, 0.5 + 2e-5, 0.0, np.nan, 4.5, 2.5]]], np.float32)   # d_aff 1, 1e-5, -, -, 2, 1
    c = np.array([[[1.0, 1.0, 1.0, 1.0, 0.5, 0.0]]], np.float32)
    res, gate = rf.prompt_feats(pts, d, c, [2.0], [0.5])
    ok = np.array([1, 0, 0, 0, 1, 1], bool)
    lda = np.where(ok, np.log(np.maximum(np.where(ok, (d[0, 0] - 0.5) / 2.0, 1.0), 1e-4)), logz[0])
    g = c[0, 0] * ok
    np.testing.assert_allclose(gate[0, 0], g, rtol=0, atol=0)
    np.testing.assert_allclose(res[0, 0], (lda - logz[0]) * g, rtol=1e-6, atol=1e-7)
    assert res[0, 0, 1] == 0 and res[0, 0, 2] == 0 and res[0, 0, 3] == 0      # d_aff <= 1e-4, d = 0, d = NaN
    assert res[0, 0, 5] == 0 and gate[0, 0, 5] == 0                          # conf 0: no gate
    _, soft = rf.prompt_feats(pts, d, c, [2.0], [0.5], soft_gate=True)
    np.testing.assert_allclose(soft[0, 0], (np.float32(0.15) + np.float32(0.85) * c[0, 0]) * ok, rtol=0, atol=0)
    # a vanishing scale is clamped at 1e-6 (v3.py:375): d_aff = (2.5 - 0.5) / 1e-6
    r2, _ = rf.prompt_feats(pts, d, c, [1e-9], [0.5])
    assert abs(r2[0, 0, 0] - (np.log(2.0 / 1e-6) - 0.3)) < 1e-4
    # the step feeds [residual, gate] to prompt_proj in that order: swapping the two columns changes the module
    cfg, sc, w, zq, pf = _level0(n_blocks=1)
    f = sc.points.reshape(-1, 3)
    a = rf.forward(f, zq, cfg.H, cfg.W, w, pf)
    b = rf.forward(f, zq, cfg.H, cfg.W, w, pf[:, ::-1].copy())
    assert np.abs(a - b).max() > 1e-4


def test_zero_out_proj_adds_its_bias():
    """out_proj zero with bias delta: the refined log depth is logz + delta exactly (_refine_logz, v3.py:359)."""
    cfg, sc, w, zq, pf = _level0()
    wz = dataclasses.replace(w, out_w=np.zeros_like(w.out_w), out_b=np.array([0.125], np.float32))
    pts, _, _ = rf.step(sc.points[None], sc.lidar[None], sc.conf[None], wz, precision="int8", iters=4)
    assert np.array_equal(pts[..., 2], sc.points[None, ..., 2] + np.float32(0.125))
    assert np.array_equal(pts[..., :2], sc.points[None, ..., :2])


def test_torch_cpu_port_matches_fakequant_oracle():
    """The CPU baseline (oracle/torch_port.py: the _fallback path in torch) computes the oracle's fake-quant step:
    the same model in another fp32 order, so the same statistical bounds as the int8 comparison above."""
    from oracle import torch_port

    sc, w = _small("int8", 16, 3)
    got = torch_port.step(sc.points[None], sc.lidar[None], sc.conf[None], w, iters=10)
    ref = rf.step_fakequant(sc.points[None], sc.lidar[None], sc.conf[None], w, iters=10)
    d, dr = np.exp(got[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
    rel = np.abs(d - dr) / dr
    assert np.median(rel) < 1e-6 and rel.mean() < 1e-4 and (rel > 1e-3).mean() < 5e-3, (rel.mean(), rel.max())
    assert np.abs(got[..., 2] - sc.points[None, ..., 2]).mean() > 1e-3
