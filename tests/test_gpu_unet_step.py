"""GPU parity of the fused multi-level refine step (UNetStep / pmg_unet_step, csrc/pmg_unet.hip) against the oracle's
composition (oracle/unet.py: step), on identical seeded inputs.

The step is v3.py:547-576 around Sparse3DUNet (sparse_unet.py:176-258): prompt fit -> (residual, gate) -> _voxelize
-> U-Net -> logz + delta (output gate) -> elastic anchor -> final fit -> post_depth, one captured graph. The device's
prompt and anchor fits are checked against the fp64 oracle fit within 1e-5 and then handed to the oracle
(st_given), so that everything after a fit is compared bit for bit: the refined point map and post_depth (with the
device's final fit, itself within 1e-5 of the oracle's).
"""
import functools

import numpy as np
import pytest
import torch

from oracle import fit as ofit
from oracle import refiner as orf
from oracle import structure as ost
from oracle import unet as ou
from promptmoge_amd import spec
from promptmoge_amd import unet_weights as uw
from promptmoge_amd.unet import UNetStep

from conftest import announce

pytestmark = pytest.mark.gpu

CH = [32, 64, 128, 256, 256]  # the deployed (narrowed) Model A / B refiner widths, train.py:124
ENC = 1024
ITERS = 10


def _scene(H, W, seed=7):
    cfg = spec.StepConfig("u", H, W, 0.9 * W, 0.9 * W, W / 2, H / 2, CH[0], 1, "int8", seed=seed)
    sc = spec.make_scene(cfg)
    rng = np.random.default_rng(seed)
    enc = rng.normal(0, 1, (1, ENC, H // 16, W // 16)).astype(np.float32)
    bias = rng.normal(0, 0.1, (1, CH[-1], H // 16, W // 16)).astype(np.float32)
    return sc.points[None].copy(), sc.lidar[None].copy(), sc.conf[None].copy(), enc, bias


@functools.lru_cache(maxsize=1)
def _weights():
    """Synthetic 5-level weights with activation clips calibrated on the 240 x 320 scene (any positive clips give a
    valid int8 refiner; calibrating keeps the activations in range)."""
    w = uw.make_unet_weights(CH, ENC, enc_blocks=[1] * 5, dec_blocks=[1] * 4, bottleneck_blocks=1, seed=7)
    pts, lid, cnf, enc, bias = _scene(240, 320)
    z, tg, m, d, c = ofit.prompt_inputs(pts, lid, cnf)
    st = ofit.fit_f64(z, tg, m, ITERS)
    r, g = orf.prompt_feats(pts, d, c, st[0], st[1])
    pf = np.stack([r.reshape(-1), g.reshape(-1)], 1)
    zq, coords, zext, _ = ost.voxelize(pts)
    levels = ou.build_levels(coords, (1, 240, 320, zext), w.factors, zkeys=zq)
    return ou.calibrate(w, levels, pts.reshape(-1, 3), enc, pf, bias)


def _close_st(s, t, so, to, tol=1e-5):
    assert abs(float(s) - float(so)) <= tol * abs(float(so)), (s, so)
    assert abs(float(t) - float(to)) <= tol * max(abs(float(to)), 1.0), (t, to)


CASES = {
    # name: (H, W, output_gate, anchor)
    "modelB5": (240, 320, False, 0.0),
    "modelB5_gate_anchor": (240, 320, True, 0.3),
    "modelA5_gate_anchor": (480, 640, True, 0.3),
}


@pytest.mark.parametrize("name", list(CASES))
def test_unet_step_matches_oracle(gpu, name):
    H, W, gate, anchor = CASES[name]
    announce(f"unet step case={name} ({H}x{W}, 5 levels, gate={gate}, anchor={anchor})")
    w = _weights()
    pts, lid, cnf, enc, bias = _scene(H, W)
    step = UNetStep(w, 1, H, W, fit_iters=ITERS, final_fit=True, post_depth=True, output_gate=gate, anchor=anchor,
                    device=gpu)
    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
        P, L, Cf, E, Bm = t(pts), t(lid), t(cnf), t(enc), t(bias)
        out = torch.empty_like(P)
        st, fin = step(P, L, Cf, E, Bm, out=out)
        step.check()
        got, st, fin = out.cpu().numpy(), st.cpu().numpy(), fin.cpu().numpy()
        depth = step.depth.cpu().numpy()
        st_a = step.anchor_fit().cpu().numpy() if anchor else None
        # a replay of the captured graph repeats the step bit for bit
        out2 = torch.empty_like(P)
        step(P, L, Cf, E, Bm, out=out2)
        step.check()
        assert torch.equal(out, out2)
    # the device's prompt fit against the fp64 oracle fit
    z, tg, m, _, _ = ofit.prompt_inputs(pts, lid, cnf)
    so, to = ofit.fit_f64(z, tg, m, ITERS)
    _close_st(st[0, 0], st[0, 1], so[0], to[0])
    trace = {}
    ref, _, fin_o, _ = ou.step(pts, lid, cnf, w, enc, bias, iters=ITERS, final_fit=True, output_gate_on=gate,
                               gate_floor=0.1, anchor=anchor, st_given=(st[:, 0], st[:, 1]),
                               st_anchor_given=None if st_a is None else (st_a[:, 0], st_a[:, 1]), trace=trace)
    if anchor:
        za, tga, ma, _, _ = ofit.prompt_inputs(trace["before_anchor"], lid, cnf)
        sa, ta = ofit.fit_f64(za, tga, ma, ITERS)
        _close_st(st_a[0, 0], st_a[0, 1], sa[0], ta[0])
    assert np.array_equal(got, ref), np.abs(got - ref).max()
    _close_st(fin[0, 0], fin[0, 1], fin_o[0][0], fin_o[1][0])
    dref = ofit.post_depth(ref, (fin[:, 0], fin[:, 1]))
    assert np.array_equal(depth.view(np.uint32), dref.view(np.uint32))
    # the step moved the depth, and the prompt entered it
    assert np.abs(ref[..., 2] - pts[..., 2]).max() > 1e-3
    assert np.abs(trace["prompt_feats"][:, 1]).max() > 0.5


def test_unet_step_in_place_k2(gpu):
    """Two steps in place (points_out = points, the loop's current_coord update, v3.py:574) with the prompt fit
    re-run on the refined map each time, against two oracle steps."""
    announce("unet step K=2 in place, 240x320")
    w = _weights()
    pts, lid, cnf, enc, bias = _scene(240, 320, seed=9)
    step = UNetStep(w, 1, 240, 320, fit_iters=ITERS, final_fit=False, device=gpu)
    s = torch.cuda.Stream(gpu)
    cur = pts
    with torch.cuda.stream(s):
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
        P, L, Cf, E, Bm = t(pts), t(lid), t(cnf), t(enc), t(bias)
        for k in range(2):
            st, fin = step(P, L, Cf, E, Bm)
            step.check()
            assert fin is None
            st = st.cpu().numpy()
            z, tg, m, _, _ = ofit.prompt_inputs(cur, lid, cnf)
            so, to = ofit.fit_f64(z, tg, m, ITERS)
            _close_st(st[0, 0], st[0, 1], so[0], to[0])
            cur, _, _, _ = ou.step(cur, lid, cnf, w, enc, bias, iters=ITERS, st_given=(st[:, 0], st[:, 1]))
            assert np.array_equal(P.cpu().numpy(), cur), k
