"""GPU parity at the full sizes of the benchmark configurations.

  T  teacher fp16, 480 x 640, C = 64, K = 3 (structure rebuilt every step): each step's refined depth within 1e-3
     relative of the oracle step on the same input, with the device's prompt fit (itself within 1e-5 of the fp64 fit)
  H  int8, 756 x 1008, C = 64, K = 3, planes + thin cylinders, 20 % LiDAR holes filled on the device
     (nearest_fill): the fill bit-exact, each prompt fit and the final fit within 1e-5, and -- given the device's
     (s, t) -- the refined point map bit-exact at every step
  U  the 1M-voxel conv microbench set: the hash map bit-exact against the sorted map over all 27 x 1M entries, the
     int8 convolution with per-channel requantisation bit-exact on 65,536 sampled rows at C = 64 and 128, and the
     benchmarked mask-sorted (ordered) convolution identical to it on every row
"""
import numpy as np
import pytest
import torch

from oracle import conv as ocv
from oracle import fill as ofl
from oracle import fit as ofit
from oracle import refiner as orf
from oracle import structure as ost
from promptmoge_amd import ops, spec
from promptmoge_amd.refiner import RefinerStep

from conftest import announce

pytestmark = pytest.mark.gpu


def _fit_close(st, z, tg, m, iters):
    so, to = ofit.fit_f64(z, tg, m, iters)
    for b in range(st.shape[0]):
        assert abs(st[b, 0] - so[b]) <= 1e-5 * abs(so[b]) and abs(st[b, 1] - to[b]) <= 1e-5 * max(1.0, abs(to[b]))


def _k_steps(cfg, sc, w, lidar, conf, dev, exact: bool):
    step = RefinerStep(w, 1, cfg.H, cfg.W, precision=cfg.precision, fit_iters=cfg.fit_iters, final_fit=True)
    pts = sc.points[None].copy()
    ref = pts.copy()
    with torch.cuda.stream(torch.cuda.Stream()):
        L, Cf = torch.from_numpy(lidar[None]).to(dev), torch.from_numpy(conf[None]).to(dev)
        P = torch.from_numpy(pts).to(dev)
        for k in range(cfg.steps):
            announce(f"config {cfg.name} step {k + 1}/{cfg.steps}")
            before = P.cpu().numpy()
            st, fin = step(P, L, Cf)
            step.check()
            got, st, fin = P.cpu().numpy(), st.cpu().numpy(), fin.cpu().numpy()
            z, tg, m, _, _ = ofit.prompt_inputs(before, lidar[None], conf[None])
            _fit_close(st, z, tg, m, cfg.fit_iters)
            # the oracle step on the same input (exact: the oracle's own chain, which stays identical)
            src = ref if exact else before
            ref, _, _ = orf.step(src, lidar[None], conf[None], w, precision=cfg.precision, iters=cfg.fit_iters,
                                 st_given=(st[:, 0], st[:, 1]))
            if exact:
                assert np.array_equal(got, ref), f"step {k + 1}"
            else:
                d, dr = np.exp(got[..., 2].astype(np.float64)), np.exp(ref[..., 2].astype(np.float64))
                assert (np.abs(d - dr) / dr).max() < 1e-3, f"step {k + 1}"
            zf, tf, mf = ofit.final_inputs(got, lidar[None], conf[None])
            _fit_close(fin, zf, tf, mf, cfg.fit_iters)
            assert np.abs(got[..., 2] - before[..., 2]).mean() > 1e-4  # the step moved the depth
    return got


def test_teacher_T_three_steps(gpu):
    cfg = spec.CONFIGS["T"]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    _k_steps(cfg, sc, w, sc.lidar, sc.conf, gpu, exact=False)


def test_hires_H_three_steps_with_device_fill(gpu):
    cfg = spec.CONFIGS["H"]
    raw = spec.make_scene(cfg, fill=False)
    assert (raw.lidar == 0).mean() > 0.19
    announce("config H nearest_fill 756x1008, 20 % holes")
    d_t, c_t = ops.nearest_fill(torch.from_numpy(raw.lidar).to(gpu), torch.from_numpy(raw.conf).to(gpu))
    lidar, conf = d_t.cpu().numpy(), c_t.cpu().numpy()
    ref_l, ref_c = ofl.nearest_fill(raw.lidar, raw.conf)
    assert np.array_equal(lidar, ref_l) and np.array_equal(conf, ref_c)
    w = spec.refiner_for(cfg, raw)
    _k_steps(cfg, raw, w, lidar, conf, gpu, exact=True)


@pytest.mark.parametrize("C", [64, 128])
def test_microbench_set_map_and_conv(gpu, C):
    announce(f"microbench 1M voxels: hash map and int8 QLIN conv C={C}")
    coords = spec.make_voxels(1_000_000, 1024, seed=21)
    M = coords.shape[0]
    shape = (1, 1024, 1024, 1024)
    nt, tm, nr, rm = ops.nmap_hash(torch.from_numpy(coords).to(gpu), shape, rows=True, row_mask=True)
    nmap = ost.nmap_sorted(coords, shape)
    assert np.array_equal(nt.cpu().numpy().T, nmap)
    assert np.array_equal(tm.cpu().numpy().view(np.uint32), ost.tile_masks(nmap))
    # the set is in _linearise order: the column-run map is the same map
    st, stm, snr, srm = ops.nmap_sorted(torch.from_numpy(coords).to(gpu), shape, rows=True, row_mask=True)
    assert torch.equal(st, nt) and torch.equal(stm, tm) and torch.equal(snr, nr) and torch.equal(srm, rm)
    rng = np.random.default_rng(C)
    x = rng.integers(-127, 128, size=(M, C)).astype(np.int8)
    w = rng.integers(-127, 128, size=(C, 3, 3, 3, C)).astype(np.int8)
    mult = (rng.uniform(0.5, 2.0, size=C) / (C * 27 * 127.0)).astype(np.float32)
    q = ops.spconv_i8(torch.from_numpy(x).to(gpu), nt, tm, torch.from_numpy(w).to(gpu), ops.EPI_QLIN, a_scale=1.0,
                      w_scale=torch.from_numpy(mult).to(gpu), out_mult=1.0).cpu().numpy()
    rows = np.sort(rng.choice(M, 65_536, replace=False))
    acc = ocv.conv_acc_int(x, nmap[rows], w)
    ref = ocv.epilogue_qlin(acc, 1.0, mult, None, 1.0)
    assert np.array_equal(q[rows], ref)
    # the plain per-channel requantisation written out: clamp(rint(acc * m[n]), -127, 127)
    plain = np.clip(np.rint(acc.astype(np.float32) * mult[None, :]), -127, 127).astype(np.int8)
    assert np.array_equal(ref, plain)
    assert (ref != 0).mean() > 0.3  # the codes are not all zero
    # the benchmarked path: rows in mask-sorted order, the map permuted into it -- identical codes for every row
    order, otm, nmo = ops.row_order(rm, nr)
    qo = ops.spconv_i8_ordered(torch.from_numpy(x).to(gpu), nmo, order, otm, torch.from_numpy(w).to(gpu),
                               ops.EPI_QLIN, a_scale=1.0, w_scale=torch.from_numpy(mult).to(gpu), out_mult=1.0)
    assert np.array_equal(qo.cpu().numpy(), q)
