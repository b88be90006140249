"""GPU parity of the fused refiner step (RefinerStep) against the oracle's step on the same seeded inputs.

The prompt fit must agree to 1e-5 relative (scale) / 1e-5 m (shift); the refined depth to 1e-3 relative. The int8
stages after the fit are then compared bit for bit: the oracle step is given the device's (s, t) (already checked
against the fp64 fit within 1e-5), so the voxel keys, the int8 codes, the residual stream and the refined point map
must be identical whatever the last bits of the fit.
"""
import numpy as np
import pytest
import torch

from oracle import fit as ofit
from oracle import refiner as orf
from promptmoge_amd import spec
from promptmoge_amd.refiner import RefinerStep

from conftest import announce

pytestmark = pytest.mark.gpu


def _run(cfg, sc, w, *, B=1, use_graph=True, final_fit=False, reps=1, lidar=None, **kw):
    dev = torch.device("cuda:0")
    lidar, conf = (sc.lidar, sc.conf) if lidar is None else lidar
    pts = np.broadcast_to(sc.points, (B,) + sc.points.shape).copy()
    lid = np.broadcast_to(lidar, (B,) + lidar.shape).copy()
    cnf = np.broadcast_to(conf, (B,) + conf.shape).copy()
    step = RefinerStep(w, B, cfg.H, cfg.W, dh=lid.shape[-2], dw=lid.shape[-1], precision=cfg.precision,
                       fit_iters=cfg.fit_iters, final_fit=final_fit, use_graph=use_graph, **kw)
    stream = torch.cuda.Stream()
    outs = []
    with torch.cuda.stream(stream):
        L, Cf = torch.from_numpy(lid).to(dev), torch.from_numpy(cnf).to(dev)
        for _ in range(reps):
            P = torch.from_numpy(pts).to(dev)
            st, fin = step(P, L, Cf)
            step.check()
            outs.append((P.cpu().numpy(), st.cpu().numpy().copy(), None if fin is None else fin.cpu().numpy().copy()))
    return step, pts, lid, cnf, outs


@pytest.mark.parametrize("name", ["B", "A"])
def test_step_int8(gpu, name):
    announce(f"step int8 config={name}")
    cfg = spec.CONFIGS[name]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    step, pts, lid, cnf, outs = _run(cfg, sc, w, final_fit=True)
    P, st, fin = outs[0]
    z, tg, m, _, _ = ofit.prompt_inputs(pts, lid, cnf)
    so, to = ofit.fit_f64(z, tg, m, cfg.fit_iters)
    assert abs(st[0, 0] - so[0]) <= 1e-5 * abs(so[0]) and abs(st[0, 1] - to[0]) <= 1e-5
    trace = {}
    ref, _, fin_o = orf.step(pts, lid, cnf, w, precision="int8", iters=cfg.fit_iters, final_fit=True, trace=trace,
                             st_given=(st[:, 0], st[:, 1]))
    assert np.array_equal(step.buffer("zq").cpu().numpy(), trace["zq"].reshape(-1))
    last, before = trace["blocks"][-1], trace["blocks"][-2]
    assert np.array_equal(step.buffer("q1").cpu().numpy(), last["q1"])
    assert np.array_equal(step.buffer("q2").cpu().numpy(), last["q2"])
    assert np.array_equal(step.buffer("x").cpu().numpy(), before["x"])  # residual entering the last block
    assert np.array_equal(P, ref)
    assert abs(fin[0, 0] - fin_o[0][0]) <= 1e-5 * abs(fin_o[0][0]) and abs(fin[0, 1] - fin_o[1][0]) <= 1e-5


def test_step_int8_lowres_lidar(gpu):
    """LiDAR coarser than the point map (192 x 256 under 480 x 640): the prompt fit reads it nearest-resized up,
    the final fit area-pools the refined depth down to it (v3.py:373-378, 768-778)."""
    announce("step int8 config=A lidar=192x256")
    cfg = spec.CONFIGS["A"]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    iy, ix = (np.arange(192) * cfg.H) // 192, (np.arange(256) * cfg.W) // 256
    lowres = (np.ascontiguousarray(sc.lidar[iy][:, ix]), np.ascontiguousarray(sc.conf[iy][:, ix]))
    step, pts, lid, cnf, outs = _run(cfg, sc, w, final_fit=True, lidar=lowres)
    P, st, fin = outs[0]
    ref, st_o, fin_o = orf.step(pts, lid, cnf, w, precision="int8", iters=cfg.fit_iters, final_fit=True)
    assert abs(st[0, 0] - st_o[0][0]) <= 1e-5 * abs(st_o[0][0]) and abs(st[0, 1] - st_o[1][0]) <= 1e-5
    d, dr = np.exp(P[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
    assert (np.abs(d - dr) / dr).max() < 1e-3
    assert abs(fin[0, 0] - fin_o[0][0]) <= 1e-5 * abs(fin_o[0][0]) and abs(fin[0, 1] - fin_o[1][0]) <= 1e-5


@pytest.mark.parametrize("gate,anchor", [(True, 0.0), (False, 0.5), (True, 0.3)])
def test_step_output_gate_and_anchor(gpu, gate, anchor):
    """The refine loop's 'output_gate' (floor 0.1) and elastic 'anchor' options (v3.py:565-573) in the fused step:
    refined depth within 1e-3 relative of the oracle (the anchor re-fits (s, t) on the refined depth, in fp64 sums
    of another order); with the gate alone and a bit-identical prompt fit, the depth is bit-identical."""
    announce(f"step int8 config=B output_gate={gate} anchor={anchor}")
    cfg = spec.CONFIGS["B"]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    step, pts, lid, cnf, outs = _run(cfg, sc, w, final_fit=True, output_gate=gate, output_gate_floor=0.1,
                                     anchor=anchor)
    P, st, fin = outs[0]
    ref, st_o, fin_o = orf.step(pts, lid, cnf, w, precision="int8", iters=cfg.fit_iters, final_fit=True,
                                output_gate_on=gate, gate_floor=0.1, anchor=anchor)
    plain, _, _ = orf.step(pts, lid, cnf, w, precision="int8", iters=cfg.fit_iters)
    assert abs(st[0, 0] - st_o[0][0]) <= 1e-5 * abs(st_o[0][0]) and abs(st[0, 1] - st_o[1][0]) <= 1e-5
    d, dr = np.exp(P[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
    assert (np.abs(d - dr) / dr).max() < 1e-3
    assert abs(fin[0, 0] - fin_o[0][0]) <= 1e-5 * abs(fin_o[0][0]) and abs(fin[0, 1] - fin_o[1][0]) <= 1e-5
    # the options change the result (the test would not notice a step that ignores them)
    assert np.abs(ref[..., 2] - plain[..., 2]).max() > 1e-4
    if not anchor and st[0, 0] == st_o[0][0] and st[0, 1] == st_o[1][0]:
        assert np.array_equal(P, ref)


def test_step_batch_of_distinct_frames(gpu):
    """B = 2 different scenes through one step (per-frame fits, batch-offset LiDAR lookups in the gate and the
    anchor) against the oracle on the same batch."""
    announce("step int8 B=2 distinct frames, output gate + anchor")
    cfg = spec.CONFIGS["B"]
    sc0, sc1 = spec.make_scene(cfg), spec.make_scene(cfg, seed=cfg.seed + 17)
    w = spec.refiner_for(cfg, sc0)
    dev = torch.device("cuda:0")
    pts = np.stack([sc0.points, sc1.points])
    lid, cnf = np.stack([sc0.lidar, sc1.lidar]), np.stack([sc0.conf, sc1.conf])
    step = RefinerStep(w, 2, cfg.H, cfg.W, fit_iters=cfg.fit_iters, final_fit=True, output_gate=True, anchor=0.25)
    with torch.cuda.stream(torch.cuda.Stream()):
        P = torch.from_numpy(pts).to(dev)
        st, fin = step(P, torch.from_numpy(lid).to(dev), torch.from_numpy(cnf).to(dev))
        step.check()
        got, st, fin = P.cpu().numpy(), st.cpu().numpy(), fin.cpu().numpy()
    ref, st_o, fin_o = orf.step(pts, lid, cnf, w, precision="int8", iters=cfg.fit_iters, final_fit=True,
                                output_gate_on=True, gate_floor=0.1, anchor=0.25)
    for b in range(2):
        assert abs(st[b, 0] - st_o[0][b]) <= 1e-5 * abs(st_o[0][b]) and abs(st[b, 1] - st_o[1][b]) <= 1e-5
        assert abs(fin[b, 0] - fin_o[0][b]) <= 1e-5 * abs(fin_o[0][b]) and abs(fin[b, 1] - fin_o[1][b]) <= 1e-5
    d, dr = np.exp(got[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
    assert (np.abs(d - dr) / dr).max() < 1e-3
    assert np.abs(pts[0, ..., 2] - pts[1, ..., 2]).max() > 0.1  # two different scenes


def test_step_odd_sizes(gpu):
    """A 61 x 83 point map (no dimension a multiple of anything the kernels tile by), B = 3 frames, C = 32, a
    29 x 41 LiDAR grid (fractional nearest / area windows), output gate and anchor on: every stage against the
    oracle."""
    announce("step int8 61x83 B=3 C=32, LiDAR 29x41, gate + anchor")
    cfg = spec.StepConfig("odd", 61, 83, 70.0, 70.0, 41.0, 30.0, 32, 2, "int8", seed=23)
    scs = [spec.make_scene(cfg, seed=23 + 5 * k) for k in range(3)]
    w = spec.refiner_for(cfg, scs[0])
    iy, ix = (np.arange(29) * cfg.H) // 29, (np.arange(41) * cfg.W) // 41
    pts = np.stack([sc.points for sc in scs])
    lid = np.stack([np.ascontiguousarray(sc.lidar[iy][:, ix]) for sc in scs])
    cnf = np.stack([np.ascontiguousarray(sc.conf[iy][:, ix]) for sc in scs])
    dev = torch.device("cuda:0")
    step = RefinerStep(w, 3, cfg.H, cfg.W, dh=29, dw=41, fit_iters=cfg.fit_iters, final_fit=True, output_gate=True,
                       output_gate_floor=0.2, anchor=0.4)
    with torch.cuda.stream(torch.cuda.Stream()):
        P = torch.from_numpy(pts).to(dev)
        st, fin = step(P, torch.from_numpy(lid).to(dev), torch.from_numpy(cnf).to(dev))
        step.check()
        got, st, fin = P.cpu().numpy(), st.cpu().numpy(), fin.cpu().numpy()
    ref, st_o, fin_o = orf.step(pts, lid, cnf, w, precision="int8", iters=cfg.fit_iters, final_fit=True,
                                output_gate_on=True, gate_floor=0.2, anchor=0.4)
    for b in range(3):
        assert abs(st[b, 0] - st_o[0][b]) <= 1e-5 * abs(st_o[0][b]) and abs(st[b, 1] - st_o[1][b]) <= 1e-5
        assert abs(fin[b, 0] - fin_o[0][b]) <= 1e-5 * abs(fin_o[0][b]) and abs(fin[b, 1] - fin_o[1][b]) <= 1e-5
    d, dr = np.exp(got[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
    assert (np.abs(d - dr) / dr).max() < 1e-3


def test_step_fp16_teacher(gpu):
    announce("step fp16 teacher (small)")
    cfg = spec.StepConfig("t", 120, 160, 130.0, 130.0, 80.0, 60.0, 64, 3, "fp16", seed=13)
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    step, pts, lid, cnf, outs = _run(cfg, sc, w)
    P, st, _ = outs[0]
    ref, st_o, _ = orf.step(pts, lid, cnf, w, precision="fp16", iters=cfg.fit_iters)
    d, dr = np.exp(P[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
    assert (np.abs(d - dr) / dr).max() < 1e-3


def test_step_graph_replays_match_eager(gpu):
    announce("step graph replay vs eager, B=2")
    cfg = spec.CONFIGS["B"]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    _, _, _, _, eager = _run(cfg, sc, w, B=2, use_graph=False, final_fit=True, reps=1)
    _, _, _, _, graph = _run(cfg, sc, w, B=2, use_graph=True, final_fit=True, reps=4)
    for P, st, fin in graph:
        assert np.array_equal(P, eager[0][0]) and np.array_equal(st, eager[0][1]) and np.array_equal(fin, eager[0][2])


def test_step_multi_step_k3(gpu):
    announce("step K=3 (points move, structure rebuilt each step)")
    cfg = spec.StepConfig("k", 96, 128, 100.0, 100.0, 64.0, 48.0, 32, 2, "int8", seed=4)
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    dev = torch.device("cuda:0")
    step = RefinerStep(w, 1, cfg.H, cfg.W, fit_iters=10)
    pts = sc.points[None].copy()
    ref = pts.copy()
    with torch.cuda.stream(torch.cuda.Stream()):
        P = torch.from_numpy(pts).to(dev)
        L, Cf = torch.from_numpy(sc.lidar[None]).to(dev), torch.from_numpy(sc.conf[None]).to(dev)
        for _ in range(3):
            step(P, L, Cf)
            ref, _, _ = orf.step(ref, sc.lidar[None], sc.conf[None], w, iters=10)
        step.check()
        got = P.cpu().numpy()
    d, dr = np.exp(got[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
    assert (np.abs(d - dr) / dr).max() < 1e-3


@pytest.mark.parametrize("precision", ["int8", "fp16"])
def test_module_forward(gpu, precision):
    """FusedRefiner behind Sparse3DUNet.forward's signature (sparse_unet.py:176-258): (M, 1) deltas for given voxel
    features, level-0 coords and prompt features; int8 bit-exact against the oracle, fp16 within 1e-3 (log depth)."""
    from promptmoge_amd.refiner import FusedRefiner
    from oracle import structure as ost

    announce(f"module forward {precision}")
    cfg = spec.CONFIGS["B"] if precision == "int8" else spec.StepConfig("t", 96, 128, 100.0, 100.0, 64.0, 48.0, 64,
                                                                         3, "fp16", seed=13)
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    B, H, W = 2, cfg.H, cfg.W
    pts = np.stack([sc.points, sc.points * np.float32(1.02)])
    zq, coords, zext, _ = ost.voxelize(pts)
    M = B * H * W
    rng = np.random.default_rng(1)
    pf = np.stack([rng.normal(0, 0.05, M), rng.uniform(0, 1, M)], 1).astype(np.float32)
    feats = pts.reshape(M, 3)
    dev = torch.device("cuda:0")
    mod = FusedRefiner(w, precision=precision)
    shape = torch.Size([B, H, W, int(zext), 3])
    tf, tc, tp = (torch.from_numpy(a).to(dev) for a in (feats, coords, pf))
    out = mod(tf, tc, shape, None, prompt_feats=tp)
    out_nc = mod(tf, None, shape, None, prompt_feats=tp)     # keys from feats[:, 2]: same map
    out_np = mod(tf, tc, shape, None)                         # no prompt_proj
    again = mod(tf, tc, shape, None, prompt_feats=tp)         # graph replay
    torch.cuda.synchronize()
    ref = orf.forward(feats, zq, H, W, w, pf, precision=precision)
    ref_np = orf.forward(feats, zq, H, W, w, None, precision=precision)
    got, got_np = out.cpu().numpy()[:, 0], out_np.cpu().numpy()[:, 0]
    assert out.shape == (M, 1)
    assert np.array_equal(out.cpu().numpy(), out_nc.cpu().numpy())
    assert np.array_equal(out.cpu().numpy(), again.cpu().numpy())
    if precision == "int8":
        assert np.array_equal(got, ref) and np.array_equal(got_np, ref_np)
    else:
        assert np.abs(got - ref).max() < 1e-3 and np.abs(got_np - ref_np).max() < 1e-3
    with pytest.raises(ValueError):
        mod(tf, torch.flip(tc, [0]).contiguous(), shape, None)    # not raster order


def test_step_expired_fit_wait_is_reported_once(gpu, libpmg):
    """A device-wide wait of the prompt fit that expires (forced from the host: one poll per wait, every kernel
    still runs to its end) is reported by check() as PMG_E_DEVICE, once; the workspace repairs itself, so the
    next step is exact again. Eager enqueue: a captured graph would keep the spin limit it was captured with."""
    from promptmoge_amd import _lib

    announce("step int8 config=B with an expired fit wait, then a clean step")
    cfg = spec.CONFIGS["B"]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    dev = torch.device("cuda:0")
    step = RefinerStep(w, 1, cfg.H, cfg.W, fit_iters=cfg.fit_iters, final_fit=True, use_graph=False)
    pts = sc.points[None].copy()
    with torch.cuda.stream(torch.cuda.Stream()):
        L, Cf = torch.from_numpy(sc.lidar[None]).to(dev), torch.from_numpy(sc.conf[None]).to(dev)
        clean = torch.from_numpy(pts).to(dev)
        step(clean, L, Cf)
        step.check()
        clean = clean.cpu().numpy()
        prev = libpmg.pmg_debug_fit_spin_limit(1)
        try:
            P = torch.from_numpy(pts).to(dev)
            st, _ = step(P, L, Cf)
        finally:
            libpmg.pmg_debug_fit_spin_limit(prev)
        with pytest.raises(_lib.PmgError) as e:
            step.check()
        assert e.value.code == _lib.PMG_E_DEVICE
        assert np.isnan(st.cpu().numpy()).all()   # the racy prompt fit is not returned as a number
        step.check()                              # reported once
        P = torch.from_numpy(pts).to(dev)
        step(P, L, Cf)
        step.check()
        assert np.array_equal(P.cpu().numpy(), clean)
