"""GPU parity of each kernel family against the oracle on identical seeded inputs.

Integer outputs (voxel keys, neighbour maps, tile masks, compacted kernel maps, int32 accumulators, requantised
int8) must be bit-exact; the fp32 quantities that feed a rounding (exp, log, SiLU, LayerNorm) are bit-exact too,
because the kernels and the oracle run the same operation sequence. Tolerances, where used, are written in the test.
"""
import numpy as np
import pytest
import torch

from oracle import conv as ocv
from oracle import fit as ofit
from oracle import numerics as onm
from oracle import structure as ost
from promptmoge_amd import ops, spec

from conftest import announce

pytestmark = pytest.mark.gpu



def _assert_f16_ulp(got, ref, min_equal=0.99):
    """fp16 SiLU outputs (the kernels' silu_fast, hardware exp2 and reciprocal): every value is the correctly
    rounded fp16 of the exact silu_f32 or its neighbour (at most 1 ulp; +0 and -0 count as equal), and at least
    `min_equal` of them are identical -- the neighbours come from rounding ties of fp16 between the two forms."""
    def key(u):
        u = u.view(np.uint16).astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7FFF), u & 0x7FFF)
    d = np.abs(key(np.asarray(got)) - key(np.asarray(ref)))
    assert d.max() <= 1, int(d.max())
    assert (d == 0).mean() >= min_equal, float((d == 0).mean())

def _t(a, dev, dt=None):
    t = torch.as_tensor(np.ascontiguousarray(a))
    return t.to(device=dev, dtype=dt) if dt is not None else t.to(dev)


def _scene(name="B"):
    cfg = spec.CONFIGS[name]
    return cfg, spec.make_scene(cfg)


# ---------------------------------------------------------------------------------------------------------- math
@pytest.mark.parametrize("op", [0, 1, 2])
def test_math_bits(gpu, op):
    announce(f"math op={op}")
    x = np.logspace(-4, 6, 200_001).astype(np.float32) if op == 1 else np.linspace(-90, 90, 200_001, dtype=np.float32)
    got = ops.math_device(op, _t(x, gpu)).cpu().numpy()
    ref = [onm.exp_f32, onm.log_f32, onm.silu_f32][op](x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _near_tie_inputs():
    """(y, mult) pairs whose silu(y) * mult lies within a few ulps of every rounding tie k + 1/2 (k in -1..127):
    float64 bisection for the exact preimage on each monotone branch of SiLU, then +-12 float32 ulps around it."""
    ys, ms = [], []
    for clip in (0.37, 1.0, 3.2, 11.0):
        mult = np.float32(127.0) / np.float32(clip)
        for k in range(-1, 128):
            target = (k + 0.5) / float(mult)
            branches = [(0.0, 200.0)] if target > 0 else [(-1.2784645, 0.0), (-60.0, -1.2784645)]
            for lo, hi in branches:
                f = lambda y: y / (1.0 + np.exp(-y)) - target
                if f(lo) * f(hi) > 0:
                    continue
                a, b = lo, hi
                for _ in range(200):
                    mid = 0.5 * (a + b)
                    if (f(a) <= 0) == (f(mid) <= 0):
                        a = mid
                    else:
                        b = mid
                y0 = np.float32(0.5 * (a + b))
                bits = np.array([y0], np.float32).view(np.int32)[0]
                for d in range(-12, 13):
                    ys.append(np.array([bits + d], np.int32).view(np.float32)[0])
                    ms.append(mult)
    return np.array(ys, np.float32), np.array(ms, np.float32)


def test_silu_quant_fast_path_is_bit_exact(gpu):
    """The epilogues' SiLU requant (hardware exp2/rcp + exact re-evaluation near ties) equals the oracle's exact
    quant_i8(silu_f32(y), mult) on adversarial near-tie inputs, special values and a dense random sweep."""
    announce("silu quant fast path")
    yt, mt = _near_tie_inputs()
    rng = np.random.default_rng(7)
    yr = rng.normal(0.0, 6.0, 2_000_000).astype(np.float32)
    mr = (np.float32(127.0) / rng.uniform(0.2, 20.0, yr.size).astype(np.float32)).astype(np.float32)
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.0, -88.0, 87.5, -87.5, 1e30, -1e30, 1e-40, -1e-40],
                  np.float32)
    y = np.concatenate([yt, yr, sp, sp])
    m = np.concatenate([mt, mr, np.full(sp.size, 42.3, np.float32), np.full(sp.size, 1e6, np.float32)])
    got = ops.math_device(3, _t(np.stack([y, m], 1), gpu)).cpu().numpy()
    ref = onm.quant_i8(onm.silu_f32(y), m).astype(np.float32)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, (y[bad[:5]], m[bad[:5]], got[bad[:5]], ref[bad[:5]])
    # the near-tie set really sits on ties: most of it takes the exact path
    v = onm.silu_f32(yt).astype(np.float64) * mt
    assert np.median(np.abs(np.abs(v - np.rint(v)) - 0.5)) < 1e-4


# ---------------------------------------------------------------------------------------------------------- structure
@pytest.mark.parametrize("name", ["B", "A"])
def test_voxelize_and_column_map(gpu, name):
    announce(f"voxelize+column map config={name}")
    cfg, sc = _scene(name)
    pts = np.stack([sc.points, sc.points * np.float32(1.001)])  # B = 2
    zq_o, coords_o, Z_o, zmin_o = ost.voxelize(pts)
    nm_o = ost.nmap_column(zq_o)
    P = _t(pts, gpu)
    zq, zmin, zmax = ops.voxelize(P[..., 2:], 256.0, stride=3, shape=pts.shape[:3])
    nt, tm, nr, cd = ops.nmap_column(zq, zmin, taps=True, rows=True, coords=True)
    torch.cuda.synchronize()
    assert np.array_equal(zq.cpu().numpy(), zq_o)
    assert np.array_equal(zmin.cpu().numpy(), zmin_o)
    assert int((zmax - zmin).max()) + 1 == Z_o
    assert np.array_equal(nr.cpu().numpy(), nm_o)
    assert np.array_equal(nt.cpu().numpy(), nm_o.T)
    assert np.array_equal(cd.cpu().numpy(), coords_o)
    assert np.array_equal(tm.cpu().numpy().view(np.uint32), ost.tile_masks(nm_o))


@pytest.mark.parametrize("seed", [0, 1])
def test_hash_map_generic(gpu, seed):
    announce(f"hash map generic seed={seed}")
    rng = np.random.default_rng(seed)
    shape = (2, 40, 50, 60)
    allc = np.stack(np.meshgrid(*[np.arange(s) for s in shape], indexing="ij"), -1).reshape(-1, 4)
    coords = allc[rng.random(allc.shape[0]) < 0.15].astype(np.int32)
    coords = coords[rng.permutation(coords.shape[0])]          # caller's order, not sorted
    ref = ost.nmap_sorted(coords, shape)
    nt, tm, nr = ops.nmap_hash(_t(coords, gpu), shape, taps=True, rows=True)
    torch.cuda.synchronize()
    assert np.array_equal(nr.cpu().numpy(), ref)
    assert np.array_equal(nt.cpu().numpy(), ref.T)
    assert np.array_equal(tm.cpu().numpy().view(np.uint32), ost.tile_masks(ref))


def test_hash_map_duplicates_and_edges(gpu):
    """A duplicated coordinate resolves to one of its rows (coords are unique in a sparse tensor; the reference's
    unstable sort leaves the choice open too); voxels on every face and corner of a shape whose extents are not
    multiples of the 4-cell brick; two batch items."""
    announce("hash map duplicates and edges")
    rng = np.random.default_rng(3)
    shape = (2, 9, 6, 7)
    allc = np.stack(np.meshgrid(*[np.arange(s) for s in shape], indexing="ij"), -1).reshape(-1, 4)
    base = allc[rng.random(allc.shape[0]) < 0.5]
    dup = base[rng.integers(0, base.shape[0], 200)]
    coords = np.concatenate([base, dup])[rng.permutation(base.shape[0] + 200)].astype(np.int32)
    rows = {}
    for i, c in enumerate(map(tuple, coords)):
        rows.setdefault(c, set()).add(i)
    delta = ost.kernel_delta(1)
    nt, tm, nr = ops.nmap_hash(_t(coords, gpu), shape, taps=True, rows=True)
    torch.cuda.synchronize()
    got = nr.cpu().numpy()
    present = np.zeros_like(got, dtype=bool)
    for i, c in enumerate(coords):
        for v in range(27):
            q = tuple(int(a) for a in (c + delta[v]))
            inb = all(0 <= q[d] < shape[d] for d in range(4))
            cand = rows.get(q) if inb else None
            present[i, v] = cand is not None
            assert (got[i, v] in cand) if cand else got[i, v] == -1, (i, v)
    # the same coordinate always resolves to the same row within one map
    key_row = {}
    for i, c in enumerate(coords):
        for v in range(27):
            if got[i, v] >= 0:
                q = tuple(int(a) for a in (c + delta[v]))
                assert key_row.setdefault(q, got[i, v]) == got[i, v]
    assert np.array_equal(nt.cpu().numpy(), got.T)
    assert np.array_equal(tm.cpu().numpy().view(np.uint32), ost.tile_masks(np.where(present, 0, -1)))


def test_hash_map_surface_voxels(gpu):
    announce("hash map surface voxels 200k")
    coords = spec.make_voxels(200_000, grid=512, seed=5)
    shape = (1, 512, 512, 512)
    ref = ost.nmap_sorted(coords, shape)
    nt, tm, _ = ops.nmap_hash(_t(coords, gpu), shape)
    torch.cuda.synchronize()
    assert np.array_equal(nt.cpu().numpy(), ref.T)
    occ = (ref >= 0).sum(1).mean()
    assert 6 <= occ <= 16, occ  # surface-like occupancy


def _lin_sorted(coords, shape):
    """coords in increasing _linearise order (_core.py:89-94)."""
    key = np.zeros(coords.shape[0], np.int64)
    for d in range(4):
        key = key * shape[d] + coords[:, d]
    return coords[np.argsort(key, kind="stable")]


@pytest.mark.parametrize("seed", [0, 1])
def test_sorted_map_generic(gpu, seed):
    """nmap_sorted on a sorted set equals the oracle's sorted map (rows, taps, tile and row masks), with voxels on
    every face of a shape and two batch items."""
    announce(f"sorted map generic seed={seed}")
    rng = np.random.default_rng(seed)
    shape = (2, 40, 50, 60)
    allc = np.stack(np.meshgrid(*[np.arange(s) for s in shape], indexing="ij"), -1).reshape(-1, 4)
    coords = _lin_sorted(allc[rng.random(allc.shape[0]) < 0.15].astype(np.int32), shape)
    ref = ost.nmap_sorted(coords, shape)
    nt, tm, nr, rm = ops.nmap_sorted(_t(coords, gpu), shape, taps=True, rows=True, row_mask=True)
    torch.cuda.synchronize()
    assert np.array_equal(nr.cpu().numpy(), ref)
    assert np.array_equal(nt.cpu().numpy(), ref.T)
    assert np.array_equal(tm.cpu().numpy().view(np.uint32), ost.tile_masks(ref))
    bits = ((ref >= 0).astype(np.uint64) << np.arange(27, dtype=np.uint64)).sum(1).astype(np.uint32)
    assert np.array_equal(rm.cpu().numpy().view(np.uint32), bits)


def test_sorted_map_long_columns_stale_table_and_order_check(gpu):
    """Columns of up to 200 voxels (the binary search of the run), a workspace reused by a second, different set
    (its table entries from the first set must not be trusted), and an unsorted set, which the device check
    reports through the sticky status word."""
    announce("sorted map long columns, stale table, order check")
    rng = np.random.default_rng(7)
    shape = (1, 24, 20, 200)
    ws = ops.sorted_workspace(shape, gpu)
    sets = []
    for dens in (0.9, 0.3):
        allc = np.stack(np.meshgrid(*[np.arange(s) for s in shape], indexing="ij"), -1).reshape(-1, 4)
        keep = rng.random(allc.shape[0]) < dens * (allc[:, 1] % 3 != 1)  # some columns empty, others dense
        sets.append(_lin_sorted(allc[keep].astype(np.int32), shape))
    for coords in sets:
        ref = ost.nmap_sorted(coords, shape)
        nt, tm, nr = ops.nmap_sorted(_t(coords, gpu), shape, rows=True, workspace=ws)
        torch.cuda.synchronize()
        assert np.array_equal(nr.cpu().numpy(), ref)
        assert np.array_equal(tm.cpu().numpy().view(np.uint32), ost.tile_masks(ref))
    assert ops.sorted_status(ws) == 0
    bad = sets[1].copy()
    bad[[10, 11]] = bad[[11, 10]]
    ops.nmap_sorted(_t(bad, gpu), shape, workspace=ws)
    assert ops.sorted_status(ws) == 1
    with pytest.raises(ValueError, match="increasing"):
        ops.nmap_sorted(_t(bad, gpu), shape)


def test_kmap_and_rows(gpu):
    announce("kmap compact + nmap_from_rows")
    cfg, sc = _scene("B")
    zq_o, _, _, _ = ost.voxelize(sc.points[None])
    nm = ost.nmap_column(zq_o)
    off_o, out_o, in_o = ost.kmap_compact(nm)
    nt, tm = ops.nmap_from_rows(_t(nm, gpu))
    off, out_rows, in_rows = ops.kmap_compact(nt)
    assert np.array_equal(nt.cpu().numpy(), nm.T)
    assert np.array_equal(tm.cpu().numpy().view(np.uint32), ost.tile_masks(nm))
    assert np.array_equal(off.cpu().numpy(), off_o)
    assert np.array_equal(out_rows.cpu().numpy(), out_o) and np.array_equal(in_rows.cpu().numpy(), in_o)


# ---------------------------------------------------------------------------------------------------------- conv
def _map_from_scene(gpu, H=96, W=128, seed=3):
    cfg = spec.StepConfig("c", H, W, 100.0, 100.0, W / 2, H / 2, 16, 1, "int8", seed=seed)
    sc = spec.make_scene(cfg)
    zq_o, _, _, _ = ost.voxelize(sc.points[None])
    nm = ost.nmap_column(zq_o)
    nt, tm = ops.nmap_from_rows(_t(nm, gpu))
    return nm, nt, tm


@pytest.mark.parametrize("Ci,Co", [(16, 16), (32, 32), (48, 48), (64, 64), (128, 128), (32, 96), (48, 16)])
def test_conv_int8_accumulator(gpu, Ci, Co):
    announce(f"conv int8 acc Ci={Ci} Co={Co}")
    rng = np.random.default_rng(Ci * 1000 + Co)
    nm, nt, tm = _map_from_scene(gpu)
    M = nm.shape[0]
    x = rng.integers(-127, 128, size=(M, Ci)).astype(np.int8)
    w = rng.integers(-127, 128, size=(Co, 3, 3, 3, Ci)).astype(np.int8)
    acc = ops.spconv_i8(_t(x, gpu), nt, tm, _t(w, gpu), ops.EPI_ACC)
    assert np.array_equal(acc.cpu().numpy(), ocv.conv_acc_int(x, nm, w))


def test_conv_int8_generic_map(gpu):
    announce("conv int8 acc on a hash map")
    rng = np.random.default_rng(9)
    coords = spec.make_voxels(60_000, grid=256, seed=8)
    shape = (1, 256, 256, 256)
    nm = ost.nmap_sorted(coords, shape)
    nt, tm, _ = ops.nmap_hash(_t(coords, gpu), shape)
    x = rng.integers(-127, 128, size=(coords.shape[0], 64)).astype(np.int8)
    w = rng.integers(-127, 128, size=(64, 3, 3, 3, 64)).astype(np.int8)
    acc = ops.spconv_i8(_t(x, gpu), nt, tm, _t(w, gpu), ops.EPI_ACC)
    assert np.array_equal(acc.cpu().numpy(), ocv.conv_acc_int(x, nm, w))


def test_row_order_is_a_stable_sort_by_mask(gpu):
    """pmg_row_order: a permutation sorting the rows of each window stably by their whole 27-bit tap mask, the tile
    unions of that order, and the tap-major map permuted into it; the hash's row masks are the bits of its map rows.
    200,001 rows end in a ragged window, a ragged tile and a ragged radix tile."""
    announce("row order 200k surface voxels")
    coords = spec.make_voxels(200_001, grid=512, seed=5)
    shape = (1, 512, 512, 512)
    nt, tm, nr, rm = ops.nmap_hash(_t(coords, gpu), shape, rows=True, row_mask=True)
    order, otm, nmo = ops.row_order(rm, nr, window=65536)
    torch.cuda.synchronize()
    rows = nr.cpu().numpy()
    masks = ((rows >= 0).astype(np.uint64) << np.arange(27, dtype=np.uint64)).sum(1).astype(np.uint32)
    assert np.array_equal(rm.cpu().numpy().view(np.uint32), masks)
    win = 65536
    expect = np.concatenate([s + np.argsort(masks[s:s + win], kind="stable") for s in range(0, len(masks), win)])
    assert np.array_equal(order.cpu().numpy(), expect)
    m = masks[expect]
    assert np.all(m[1:win] >= m[:win - 1]) and len(m) % 16 != 0 and len(m) % win != 0
    pad = np.zeros(((len(m) + 15) // 16) * 16, np.uint32)
    pad[:len(m)] = m
    assert np.array_equal(otm.cpu().numpy().view(np.uint32), np.bitwise_or.reduce(pad.reshape(-1, 16), axis=1))
    assert np.array_equal(nmo.cpu().numpy(), nt.cpu().numpy()[:, expect])
    # without a map: the same order and tile masks
    o2, otm2, none = ops.row_order(rm, window=65536)
    assert none is None and torch.equal(o2, order) and torch.equal(otm2, otm)
    # one window: the whole set sorted by mask
    o3, _, _ = ops.row_order(rm, window=0)
    assert np.array_equal(o3.cpu().numpy(), np.argsort(masks, kind="stable"))


@pytest.mark.parametrize("C", [64, 128])
def test_conv_int8_ordered_matches_unordered(gpu, C):
    """The ordered convolution (map permuted into the mask-sorted order, outputs scattered back) gives
    bit-identical results to the plain one (accumulators and every epilogue) and to the oracle."""
    announce(f"conv int8 ordered C={C}")
    rng = np.random.default_rng(C + 1)
    coords = spec.make_voxels(70_001, grid=256, seed=4)
    shape = (1, 256, 256, 256)
    nt, tm, nr, rm = ops.nmap_hash(_t(coords, gpu), shape, rows=True, row_mask=True)
    order, otm, nmo = ops.row_order(rm, nr)
    M = coords.shape[0]
    x = _t(rng.integers(-127, 128, size=(M, C)).astype(np.int8), gpu)
    w = _t(rng.integers(-127, 128, size=(C, 3, 3, 3, C)).astype(np.int8), gpu)
    sc = _t(rng.uniform(1e-5, 1e-4, C).astype(np.float32), gpu)
    b = _t(rng.normal(0, 0.05, C).astype(np.float32), gpu)
    skip = _t(rng.normal(size=(M, C)).astype(np.float32), gpu)
    kw = dict(a_scale=0.02, w_scale=sc, bias=b, out_mult=30.0)
    for epi, extra in ((ops.EPI_ACC, {}), (ops.EPI_Q, {}), (ops.EPI_R, {"skip": skip}), (ops.EPI_BIAS, {}),
                       (ops.EPI_QLIN, {})):
        a = ops.spconv_i8(x, nt, tm, w, epi, **kw, **extra)
        o = ops.spconv_i8_ordered(x, nmo, order, otm, w, epi, **kw, **extra)
        torch.cuda.synchronize()
        assert torch.equal(a, o), epi
    nm = ost.nmap_sorted(coords, shape)
    assert np.array_equal(ops.spconv_i8_ordered(x, nmo, order, otm, w).cpu().numpy(),
                          ocv.conv_acc_int(x.cpu().numpy(), nm, w.cpu().numpy()))


@pytest.mark.parametrize("C", [32, 48, 64, 128])
def test_conv_int8_epilogues(gpu, C):
    announce(f"conv int8 epilogues C={C}")
    rng = np.random.default_rng(C)
    nm, nt, tm = _map_from_scene(gpu)
    M = nm.shape[0]
    x = rng.integers(-127, 128, size=(M, C)).astype(np.int8)
    wf = rng.normal(0, 0.05, size=(C, 3, 3, 3, C)).astype(np.float32)
    q, s = spec.quantize_weight(wf)
    b = rng.normal(0, 0.05, size=C).astype(np.float32)
    a_s, o_s = np.float32(3.0 / 127), np.float32(127 / 1.7)
    skip = rng.normal(size=(M, C)).astype(np.float32)
    acc = ocv.conv_acc_int(x, nm, q)
    X, Wq, S, Bv = _t(x, gpu), _t(q, gpu), _t(s, gpu), _t(b, gpu)
    out_q = ops.spconv_i8(X, nt, tm, Wq, ops.EPI_Q, a_scale=a_s, w_scale=S, bias=Bv, out_mult=o_s)
    assert np.array_equal(out_q.cpu().numpy(), ocv.epilogue_q(acc, a_s, s, b, o_s))
    Sk = _t(skip, gpu)
    out_r = ops.spconv_i8(X, nt, tm, Wq, ops.EPI_R, a_scale=a_s, w_scale=S, bias=Bv, skip=Sk, out=Sk.clone())
    assert np.array_equal(out_r.cpu().numpy(), ocv.epilogue_r(acc, a_s, s, b, skip))
    out_b = ops.spconv_i8(X, nt, tm, Wq, ops.EPI_BIAS, a_scale=a_s, w_scale=S, bias=Bv)
    assert np.array_equal(out_b.cpu().numpy(), ocv.dequant(acc, a_s, s, b))
    out_l = ops.spconv_i8(X, nt, tm, Wq, ops.EPI_QLIN, a_scale=a_s, w_scale=S, bias=Bv, out_mult=o_s)
    assert np.array_equal(out_l.cpu().numpy(), ocv.epilogue_qlin(acc, a_s, s, b, o_s))
    # the microbenchmark's plain per-channel requantisation: q = clamp(rint(acc * m[n]), +-127)
    m = (s * np.float32(0.05)).astype(np.float32)
    out_m = ops.spconv_i8(X, nt, tm, Wq, ops.EPI_QLIN, w_scale=_t(m, gpu))
    expect = np.clip(np.rint(acc.astype(np.float32) * m[None, :]), -127, 127).astype(np.int8)
    assert np.array_equal(out_m.cpu().numpy(), expect)


@pytest.mark.parametrize("C", [32, 48, 64, 128, 256, 512])
def test_conv_f16(gpu, C):
    """fp16 features: the weight-staged kernel (C = 32 .. 512; 256 and 512 in 64-channel slices) or the generic one
    (48) against the fp64 correlation within the fp32-accumulation bound; the epilogues on the kernel's own sums."""
    announce(f"conv fp16 C={C}")
    rng = np.random.default_rng(100 + C)
    nm, nt, tm = _map_from_scene(gpu) if C <= 128 else _map_from_scene(gpu, 48, 64)
    M = nm.shape[0]
    x = rng.normal(size=(M, C)).astype(np.float16)
    w = rng.normal(0, 0.05, size=(C, 3, 3, 3, C)).astype(np.float16)
    b = rng.normal(0, 0.05, size=C).astype(np.float32)
    ref = ocv.conv_float(x.astype(np.float64), nm, w.astype(np.float64), dtype=np.float64)
    got = ops.spconv_f16(_t(x, gpu), nt, tm, _t(w, gpu), ops.EPI_ACC).cpu().numpy()
    # fp32 accumulation of exact fp16 products: error bound ~ n_terms * eps32 * sum|terms|
    bound = 27 * C * 2 ** -23 * ocv.conv_float(np.abs(x.astype(np.float64)), nm, np.abs(w.astype(np.float64)),
                                                dtype=np.float64)
    assert (np.abs(got - ref) <= bound + 1e-6).all()
    h = ops.spconv_f16(_t(x, gpu), nt, tm, _t(w, gpu), ops.EPI_SILU, bias=_t(b, gpu)).cpu().numpy()
    hr = onm.silu_f32((got + b).astype(np.float32)).astype(np.float16)  # from the kernel's own accumulator
    _assert_f16_ulp(h, hr)
    # bias and residual epilogues: fp32 additions to the same accumulator
    yb = ops.spconv_f16(_t(x, gpu), nt, tm, _t(w, gpu), ops.EPI_BIAS, bias=_t(b, gpu)).cpu().numpy()
    assert np.array_equal(yb, got + b)
    skip = rng.normal(size=(M, C)).astype(np.float32)
    yr = ops.spconv_f16(_t(x, gpu), nt, tm, _t(w, gpu), ops.EPI_R, bias=_t(b, gpu), skip=_t(skip, gpu)).cpu().numpy()
    assert np.array_equal(yr, (got + b) + skip)


@pytest.mark.parametrize("C", [32, 48, 64, 128, 256])
def test_conv_bf16(gpu, C):
    announce(f"conv bf16 C={C}")
    g = torch.Generator().manual_seed(300 + C)
    nm, nt, tm = _map_from_scene(gpu) if C <= 128 else _map_from_scene(gpu, 48, 64)
    M = nm.shape[0]
    x = torch.randn(M, C, generator=g).bfloat16()
    w = (torch.randn(C, 3, 3, 3, C, generator=g) * 0.05).bfloat16()
    b = (torch.randn(C, generator=g) * 0.05).float()
    xs, ws = x.float().numpy().astype(np.float64), w.float().numpy().astype(np.float64)
    ref = ocv.conv_float(xs, nm, ws, dtype=np.float64)
    got = ops.spconv_bf16(x.to(gpu), nt, tm, w.to(gpu), ops.EPI_ACC).cpu().numpy()
    # fp32 accumulation of exact bf16 products: error bound ~ n_terms * eps32 * sum|terms|
    bound = 27 * C * 2 ** -23 * ocv.conv_float(np.abs(xs), nm, np.abs(ws), dtype=np.float64)
    assert (np.abs(got - ref) <= bound + 1e-6).all()
    bn = b.numpy()
    yb = ops.spconv_bf16(x.to(gpu), nt, tm, w.to(gpu), ops.EPI_BIAS, bias=b.to(gpu)).cpu().numpy()
    assert np.array_equal(yb, got + bn)
    skip = torch.randn(M, C, generator=g)
    yr = ops.spconv_bf16(x.to(gpu), nt, tm, w.to(gpu), ops.EPI_R, bias=b.to(gpu), skip=skip.to(gpu)).cpu().numpy()
    assert np.array_equal(yr, (got + bn) + skip.numpy())


@pytest.mark.parametrize("Ci,Co", [(24, 32), (32, 32), (64, 64)])
def test_conv_f32(gpu, Ci, Co):
    announce(f"conv fp32 {Ci}->{Co}")
    rng = np.random.default_rng(7 + Ci)
    nm, nt, tm = _map_from_scene(gpu)
    M = nm.shape[0]
    x = rng.normal(size=(M, Ci)).astype(np.float32)
    w = rng.normal(0, 0.05, size=(Co, 3, 3, 3, Ci)).astype(np.float32)
    b = rng.normal(size=Co).astype(np.float32)
    got = ops.spconv_f32(_t(x, gpu), nt, tm, _t(w, gpu), _t(b, gpu)).cpu().numpy()
    ref = ocv.conv_float(x.astype(np.float64), nm, w.astype(np.float64), b.astype(np.float64), dtype=np.float64)
    # fp32 accumulation: error bound ~ n_terms * eps32 * sum|terms| (+ the bias)
    bound = 27 * Ci * 2 ** -23 * ocv.conv_float(np.abs(x.astype(np.float64)), nm, np.abs(w.astype(np.float64)),
                                                 np.abs(b.astype(np.float64)), dtype=np.float64)
    assert (np.abs(got - ref) <= bound + 1e-6).all()
    acc = ops.spconv_f32(_t(x, gpu), nt, tm, _t(w, gpu)).cpu().numpy()
    assert np.array_equal(got, acc + b)


# ---------------------------------------------------------------------------------------------------------- row ops
@pytest.mark.parametrize("C", [16, 32, 48, 64, 128])
def test_ln_silu(gpu, C):
    announce(f"ln_silu C={C}")
    rng = np.random.default_rng(C)
    x = rng.normal(0.2, 1.5, size=(50_000, C)).astype(np.float32)
    g = spec._f16(1 + rng.normal(0, 0.05, C))
    b = spec._f16(rng.normal(0, 0.05, C))
    s = np.float32(127 / 3.2)
    X, G, Bt = _t(x, gpu), _t(g, gpu), _t(b, gpu)
    y = onm.ln_silu(x, g, b)
    assert np.array_equal(ops.ln_silu_quant(X, G, Bt, s).cpu().numpy(), onm.quant_i8(y, s))
    _assert_f16_ulp(ops.ln_silu_f16(X, G, Bt).cpu().numpy(), y.astype(np.float16))


# ---------------------------------------------------------------------------------------------------------- fit
def _close_st(s, t, so, to, tol=1e-5):
    assert abs(float(s) - float(so)) <= tol * abs(float(so)), (s, so)
    assert abs(float(t) - float(to)) <= tol * max(abs(float(to)), 1.0), (t, to)


@pytest.mark.parametrize("iters", [0, 1, 4, 10])
def test_fit_generic(gpu, iters):
    announce(f"fit generic iters={iters}")
    rng = np.random.default_rng(iters)
    B, N = 2, 100_000
    z = rng.uniform(0.5, 6, size=(B, N)).astype(np.float32)
    t = (1.3 * z + 0.05 + rng.normal(0, 0.01, size=(B, N))).astype(np.float32)
    t = np.where(rng.random((B, N)) < 0.05, t * 2.5, t).astype(np.float32)
    m = rng.random((B, N)) < 0.7
    so, to, info_o = ofit.fit_f64(z, t, m, iters=iters, return_info=True)
    s, tt, info = ops.fit_scale_shift(_t(z, gpu), _t(t, gpu), _t(m, gpu), iters=iters, return_info=True)
    s, tt, info = s.cpu().numpy(), tt.cpu().numpy(), info.cpu().numpy()
    for b in range(B):
        _close_st(s[b], tt[b], so[b], to[b])
        assert info[b, 0] == info_o[b]["count"] and info[b, 1] == info_o[b]["k"] and info[b, 4] == 0
        if iters > 0 and s[b] == so[b] and tt[b] == to[b]:  # same (s, t) every round: the same exact k-th
            assert info[b, 3] == np.float32(info_o[b]["thr"]).view(np.int32)


@pytest.mark.parametrize("case", ["ties_all", "ties_some", "large"])
def test_fit_selection_paths(gpu, case):
    """Exercises the three ways the kernel finds the k-th residual: the bracket around the previous round's
    threshold, the two global radix passes, and the third pass when one 1024-value bin holds more than the 32768
    candidates a block keeps in LDS (exact-linear data: most residuals are exactly 0)."""
    announce(f"fit selection path {case}")
    rng = np.random.default_rng(len(case))
    N = 300_000 if case == "large" else 120_000
    if case == "ties_all":
        z = rng.integers(1, 9, size=(1, N)).astype(np.float32)
        t = (2 * z).astype(np.float32)
        t = np.where(rng.random((1, N)) < 0.05, t * 3, t).astype(np.float32)
    elif case == "ties_some":
        z = rng.uniform(0.5, 6, size=(1, N)).astype(np.float32)
        t = np.round(1.3 * z + 0.05 + rng.normal(0, 0.01, size=(1, N)), 2).astype(np.float32)
    else:
        z = rng.uniform(0.5, 6, size=(1, N)).astype(np.float32)
        t = (0.7 * z + 0.3 + rng.normal(0, 0.02, size=(1, N))).astype(np.float32)
        t = np.where(rng.random((1, N)) < 0.1, t * rng.uniform(0.3, 3, size=(1, N)), t).astype(np.float32)
    m = rng.random((1, N)) < 0.7
    so, to, info_o = ofit.fit_f64(z, t, m, iters=10, return_info=True)
    s, tt, info = ops.fit_scale_shift(_t(z, gpu), _t(t, gpu), _t(m, gpu), iters=10, return_info=True)
    s, tt, info = s.cpu().numpy(), tt.cpu().numpy(), info.cpu().numpy()
    _close_st(s[0], tt[0], so[0], to[0])
    assert info[0, 4] == 0
    if s[0] == so[0] and tt[0] == to[0]:
        assert info[0, 3] == np.float32(info_o[0]["thr"]).view(np.int32)
    # a second call reuses the workspace left by the first
    s2, t2 = ops.fit_scale_shift(_t(z, gpu), _t(t, gpu), _t(m, gpu), iters=10)
    assert s2.item() == s[0] and t2.item() == tt[0]


@pytest.mark.parametrize("case", ["relative_rule", "clamp", "ties"])
def test_fit_trim_rule_closed_form(gpu, case):
    """The hand-built trimming cases (tests/fit_cases.py): after one trim the device keeps exactly the subset the rule
    of prompt_stem.py:233-239 keeps (relative residual, 1e-3 clamp, k-th smallest, r <= thr), so (s, t) equal that
    subset's least-squares line (np.polyfit in float64). Two batch items: the case, and the case reversed."""
    import fit_cases as fc

    announce(f"fit trim rule {case}")
    z, tg, kept = getattr(fc, f"{case}_case")()[:3]
    zz = np.stack([z, z[::-1]])
    tt = np.stack([tg, tg[::-1]])
    m = np.ones_like(zz, bool)
    s, t_ = ops.fit_scale_shift(_t(zz, gpu), _t(tt, gpu), _t(m, gpu), iters=1)
    es, et = fc.lstsq_st(z, tg, kept)
    for b in range(2):
        assert abs(float(s[b]) - es) < 2e-6 and abs(float(t_[b]) - et) < 2e-6, (b, float(s[b]), es, float(t_[b]), et)


def test_fit_edge_cases(gpu):
    announce("fit edge cases")
    z = np.full((3, 5000), 2.0, np.float32)
    t = np.random.default_rng(0).uniform(1, 3, size=(3, 5000)).astype(np.float32)
    m = np.ones_like(z, bool)
    m[1, 31:] = False                      # 31 points: fallback (1, 0)
    z[2] = np.linspace(0.5, 6, 5000)       # batch 2: ordinary
    so, to = ofit.fit_f64(z, t, m, iters=4)
    s, tt = ops.fit_scale_shift(_t(z, gpu), _t(t, gpu), _t(m, gpu), iters=4)
    s, tt = s.cpu().numpy(), tt.cpu().numpy()
    assert s[1] == 1.0 and tt[1] == 0.0
    assert s[0] == 1.0  # constant z: den = 0
    for b in (0, 2):
        _close_st(s[b], tt[b], so[b], to[b])


def test_fit_expired_wait_is_reported_and_does_not_leak(gpu, libpmg):
    """A device-wide wait that expires -- forced from the host with a one-poll spin limit, so every kernel still runs
    to its end -- is reported in info[:, 4] with (s, t) = NaN for that batch item, and does not leak: the next call
    on the same workspace is exact again (the last block restores the barrier state)."""
    announce("fit expired wait, then a clean call on the same workspace")
    rng = np.random.default_rng(5)
    B, N = 2, 300_000  # 74 blocks per item
    z = rng.uniform(0.5, 6, size=(B, N)).astype(np.float32)
    t = (1.3 * z + 0.05 + rng.normal(0, 0.01, size=(B, N))).astype(np.float32)
    m = rng.random((B, N)) < 0.7
    args = (_t(z, gpu), _t(t, gpu), _t(m, gpu))
    s0, t0, i0 = (a.cpu().numpy() for a in ops.fit_scale_shift(*args, iters=10, return_info=True))
    prev = libpmg.pmg_debug_fit_spin_limit(1)
    try:
        s1, t1, i1 = ops.fit_scale_shift(*args, iters=10, return_info=True)
        torch.cuda.synchronize()
    finally:
        libpmg.pmg_debug_fit_spin_limit(prev)
    s1, t1, i1 = s1.cpu().numpy(), t1.cpu().numpy(), i1.cpu().numpy()
    assert i1[:, 4].any(), "one poll per wait: some wait must expire"
    for b in range(B):
        if i1[b, 4]:
            assert np.isnan(s1[b]) and np.isnan(t1[b])
        else:
            assert s1[b] == s0[b] and t1[b] == t0[b]
    s2, t2, i2 = (a.cpu().numpy() for a in ops.fit_scale_shift(*args, iters=10, return_info=True))
    assert (i2[:, 4] == 0).all() and (i0[:, 4] == 0).all()
    assert np.array_equal(s2, s0) and np.array_equal(t2, t0)


def _fit_trace(ws: "torch.Tensor"):
    """Block 0's round record in the fit workspace: per round the selection path code (low 3 bits: 0 bracket,
    1 bracket missed -> radix, 2 radix, 4 window, 5 bracket missed -> window, 6 window missed -> radix, 7 both
    missed -> radix; bit 3: one-value threshold) and the histogram passes; the number of rounds run."""
    tr = ws[128:128 + 4096].cpu().numpy().view(np.uint32)
    rounds = int(tr[130])
    return [(int(tr[2 * i]) & 15, (int(tr[2 * i]) >> 4) & 15) for i in range(rounds)]


def test_fit_plan_fallbacks_do_not_change_results(gpu, libpmg):
    """The selection's plan only decides how fast the exact k-th is found. With plans made wrong on purpose
    (pmg_debug_fit_plan: brackets moved off their range, windows that miss, coarse windows that need split passes)
    every fallback path runs, and (s, t) and the last threshold stay bit-identical to the normal plan's, on data
    whose threshold moves for all 10 rounds (noisy line with outliers) and on an exact line with outliers (the
    threshold collapses by many octaves after the first trim)."""
    announce("fit plan fallbacks (debug plans 1-3 against the normal plan)")
    rng = np.random.default_rng(11)
    N = 300_000
    z = rng.uniform(0.5, 6, size=(2, N)).astype(np.float32)
    t = np.empty_like(z)
    t[0] = 0.7 * z[0] + 0.3 + rng.normal(0, 0.03, size=N)
    t[0] = np.where(rng.random(N) < 0.15, t[0] * rng.uniform(0.3, 3, size=N), t[0])
    t[1] = 1.3 * z[1] + 0.05
    t[1] = np.where(rng.random(N) < 0.1, t[1] * rng.uniform(0.5, 2, size=N), t[1])
    t = t.astype(np.float32)
    m = rng.random((2, N)) < 0.8
    runs = {}
    try:
        for mode in (0, 1, 2, 3):
            libpmg.pmg_debug_fit_plan(mode)
            paths = []
            res = []
            for b in range(2):  # one item per call, so that the workspace holds that item's trace
                zb = _t(z[b:b + 1], gpu)
                s_, t_, info = ops.fit_scale_shift(zb, _t(t[b:b + 1], gpu), _t(m[b:b + 1], gpu), iters=10,
                                                   return_info=True)
                torch.cuda.synchronize()
                ws = ops._fit_workspace(0, zb.device)  # the workspace this stream's calls use
                paths.append(_fit_trace(ws))
                info = info.cpu().numpy()
                assert info[0, 4] == 0
                res.append((float(s_[0]), float(t_[0]), int(info[0, 3])))
            runs[mode] = (res, paths)
    finally:
        libpmg.pmg_debug_fit_plan(0)
    so, to, _ = ofit.fit_f64(z, t, m, iters=10, return_info=True)
    for b in range(2):
        _close_st(runs[0][0][b][0], runs[0][0][b][1], so[b], to[b])
    for mode in (1, 2, 3):
        assert runs[mode][0] == runs[0][0], (mode, runs[mode][0], runs[0][0])
    codes = {mode: {c for p in runs[mode][1] for c, _ in p} for mode in runs}
    assert 0 in codes[0] and 4 in codes[0], codes[0]  # the normal plan takes brackets and windows here
    assert 5 in codes[1], codes[1]                    # a missed bracket, then a window on the k-th's side
    assert codes[2] <= {1, 2, 6, 7}, codes[2]         # no plan ever holds the k-th: radix after every miss
    assert 6 in codes[2], codes[2]
    split = [n for p in runs[3][1] for c, n in p if c == 4]
    assert split and max(split) >= 2, runs[3][1]      # coarse windows need split passes


def _random_fit_case(rng):
    """A seeded fit problem of varied shape: size, line, noise, outlier rate and spread, mask density, targets near
    the 1e-3 clamp, ties (rounded targets), iteration count."""
    N = int(rng.choice([3_000, 40_000, 150_000, 300_000, 700_000]))
    s0, t0 = rng.uniform(0.2, 3.0), rng.uniform(-0.5, 0.5)
    z = rng.uniform(0.05, 8.0, size=N).astype(np.float32)
    t = s0 * z + t0 + rng.normal(0, rng.choice([0.0, 1e-4, 1e-2, 0.1]), size=N)
    out = rng.random(N) < rng.choice([0.0, 0.05, 0.15, 0.3])
    t = np.where(out, t * rng.uniform(0.2, 5.0, size=N), t)
    if rng.random() < 0.3:
        t = np.where(rng.random(N) < 0.05, rng.uniform(0, 2e-3, size=N), t)  # targets at the 1e-3 clamp
    if rng.random() < 0.3:
        t = np.round(t, 2)  # ties among residuals
    m = rng.random(N) < rng.choice([0.3, 0.8, 1.0])
    iters = int(rng.choice([1, 4, 10]))
    return z[None], t.astype(np.float32)[None], m[None], iters


def test_fit_random_cases_and_forced_plans(gpu, libpmg):
    """Seeded random fit problems (sizes 3k-700k, both element layouts of the kernel): (s, t) against the fp64
    oracle within 1e-5 and the threshold bit-equal when (s, t) are; and under each wrong-on-purpose plan
    (pmg_debug_fit_plan 1-3) the normal plan's (s, t) and threshold bit for bit."""
    rng = np.random.default_rng(2026)
    for case in range(12):
        z, t, m, iters = _random_fit_case(rng)
        announce(f"fit random case {case}: N={z.shape[1]} iters={iters}")
        so, to, info_o = ofit.fit_f64(z, t, m, iters=iters, return_info=True)
        res = {}
        try:
            for mode in (0, 1, 2, 3):
                libpmg.pmg_debug_fit_plan(mode)
                s_, t_, info = ops.fit_scale_shift(_t(z, gpu), _t(t, gpu), _t(m, gpu), iters=iters, return_info=True)
                info = info.cpu().numpy()
                assert info[0, 4] == 0
                res[mode] = (float(s_[0]), float(t_[0]), int(info[0, 3]))
        finally:
            libpmg.pmg_debug_fit_plan(0)
        s0_, t0_, thr0 = res[0]
        _close_st(s0_, t0_, so[0], to[0])
        if np.float32(s0_) == np.float32(so[0]) and np.float32(t0_) == np.float32(to[0]):
            assert thr0 == np.float32(info_o[0]["thr"]).view(np.int32), case
        for mode in (1, 2, 3):
            assert res[mode] == res[0], (case, mode, res[mode], res[0])


@pytest.mark.parametrize("name", ["B", "A", "H"])
def test_fit_prompt_scene(gpu, name):
    announce(f"fit prompt scene={name}")
    cfg, sc = _scene(name)
    z, tg, m, _, _ = ofit.prompt_inputs(sc.points[None], sc.lidar[None], sc.conf[None])
    so, to = ofit.fit_f64(z, tg, m, iters=10)
    s, t = ops.fit_prompt(_t(sc.points[None], gpu), _t(sc.lidar[None], gpu), _t(sc.conf[None], gpu), iters=10)
    _close_st(s.item(), t.item(), so[0], to[0])


def _lowres(sc, dh, dw):
    """The scene's LiDAR and confidence sampled down to (dh, dw), nearest: a sensor coarser than the point map."""
    H, W = sc.lidar.shape
    iy = (np.arange(dh) * H) // dh
    ix = (np.arange(dw) * W) // dw
    return np.ascontiguousarray(sc.lidar[iy][:, ix]), np.ascontiguousarray(sc.conf[iy][:, ix])


@pytest.mark.parametrize("name,dh,dw,with_mask", [("A", 192, 256, False), ("A", 192, 256, True), ("B", 240, 320, False),
                                                   ("B", 240, 320, True), ("A", 480, 640, True),
                                                   ("H", 189, 252, False)])
def test_fit_final_scene(gpu, name, dh, dw, with_mask):
    """The final metric fit (v3.py:768-778) at LiDAR resolution: area-pooled depth and the LiDAR mask."""
    announce(f"fit final scene={name} lidar={dh}x{dw} mask_binary={with_mask}")
    cfg, sc = _scene(name)
    lid, cnf = _lowres(sc, dh, dw)
    B = 2
    pts = np.stack([sc.points, sc.points * np.float32(1.01)])
    lid2, cnf2 = np.stack([lid, lid]), np.stack([cnf, cnf[::-1]])
    mb = None
    if with_mask:
        rng = np.random.default_rng(4)
        mb = rng.random((B, cfg.H, cfg.W)) > 0.002      # sparse holes: some windows fall below 0.99
    z, tg, m = ofit.final_inputs(pts, lid2, cnf2, mb)
    so, to, info_o = ofit.fit_f64(z, tg, m, iters=10, return_info=True)
    s, t, info = ops.fit_final(_t(pts, gpu), _t(lid2, gpu), _t(cnf2, gpu), None if mb is None else _t(mb, gpu),
                               iters=10, return_info=True)
    s, t, info = s.cpu().numpy(), t.cpu().numpy(), info.cpu().numpy()
    for b in range(B):
        assert info[b, 0] == info_o[b]["count"] and info[b, 4] == 0   # the mask is exact
        _close_st(s[b], t[b], so[b], to[b])


# ---------------------------------------------------------------------------------------------------------- level-0 conv
def _col_setup(gpu, H=96, W=136, seed=3, B=2):
    cfg = spec.StepConfig("c", H, W, 100.0, 100.0, W / 2, H / 2, 16, 1, "int8", seed=seed)
    sc = spec.make_scene(cfg)
    pts = np.stack([sc.points] + [sc.points * np.float32(1.0 + 0.01 * b) for b in range(1, B)])
    zq_o, _, _, _ = ost.voxelize(pts)
    nm = ost.nmap_column(zq_o)
    return pts, zq_o, nm, _t(zq_o.astype(np.int32), gpu)


@pytest.mark.parametrize("C", [16, 32, 48, 64, 128])
def test_conv_col_int8_accumulator(gpu, C):
    announce(f"conv col int8 acc C={C}")
    rng = np.random.default_rng(C + 7)
    pts, zq_o, nm, zq = _col_setup(gpu)  # W = 136: segments straddle image rows and the batch boundary
    M = nm.shape[0]
    x = rng.integers(-127, 128, size=(M, C)).astype(np.int8)
    w = rng.integers(-127, 128, size=(C, 3, 3, 3, C)).astype(np.int8)
    acc = ops.spconv_col(_t(x, gpu), zq, _t(w, gpu), ops.EPI_ACC)
    assert np.array_equal(acc.cpu().numpy(), ocv.conv_acc_int(x, nm, w))


@pytest.mark.parametrize("C", [32, 48, 128])
def test_conv_col_int8_fused_epilogues(gpu, C):
    announce(f"conv col int8 epilogues Q/R/RLN/ROUT C={C}")
    from oracle import refiner as orf

    rng = np.random.default_rng(C)
    pts, zq_o, nm, zq = _col_setup(gpu)
    M = nm.shape[0]
    x = rng.integers(-127, 128, size=(M, C)).astype(np.int8)
    q, s = spec.quantize_weight(rng.normal(0, 0.05, size=(C, 3, 3, 3, C)).astype(np.float32))
    b = rng.normal(0, 0.05, size=C).astype(np.float32)
    g = spec._f16(1 + rng.normal(0, 0.05, C))
    be = spec._f16(rng.normal(0, 0.05, C))
    a_s, o_s, n_s = np.float32(3.0 / 127), np.float32(127 / 1.7), np.float32(127 / 2.9)
    skip = rng.normal(size=(M, C)).astype(np.float32)
    acc = ocv.conv_acc_int(x, nm, q)
    X, Wq, S, Bv = _t(x, gpu), _t(q, gpu), _t(s, gpu), _t(b, gpu)
    out_q = ops.spconv_col(X, zq, Wq, ops.EPI_Q, a_scale=a_s, w_scale=S, bias=Bv, out_mult=o_s)
    assert np.array_equal(out_q.cpu().numpy(), ocv.epilogue_q(acc, a_s, s, b, o_s))
    xr = ocv.epilogue_r(acc, a_s, s, b, skip)
    out_r = ops.spconv_col(X, zq, Wq, ops.EPI_R, a_scale=a_s, w_scale=S, bias=Bv, skip=_t(skip, gpu))
    assert np.array_equal(out_r.cpu().numpy(), xr)
    Sk = _t(skip, gpu)  # RLN in place on the residual, as the step runs it
    nq = torch.empty((M, C), dtype=torch.int8, device=gpu)
    ops.spconv_col(X, zq, Wq, ops.EPI_RLN, a_scale=a_s, w_scale=S, bias=Bv, skip=Sk, out=Sk, ln_gamma=_t(g, gpu),
                   ln_beta=_t(be, gpu), next_mult=n_s, next_q=nq)
    assert np.array_equal(Sk.cpu().numpy(), xr)
    assert np.array_equal(nq.cpu().numpy(), onm.quant_i8(onm.ln_silu(xr, g, be), n_s))
    ow = rng.normal(0, 0.05, size=(1, C)).astype(np.float32)
    ob = np.array([0.01], np.float32)
    P = _t(pts, gpu)
    Po = torch.empty_like(P)
    ops.spconv_col(X, zq, Wq, ops.EPI_ROUT, a_scale=a_s, w_scale=S, bias=Bv, skip=_t(skip, gpu), out_w=_t(ow, gpu),
                   out_b=_t(ob, gpu), points=P, points_out=Po)

    class _W:
        out_w, out_b = ow, ob

    ref = pts.copy()
    ref[..., 2] = ref[..., 2] + orf.out_proj(xr, _W).reshape(ref.shape[:3])
    assert np.array_equal(Po.cpu().numpy(), ref)


@pytest.mark.parametrize("C", [32, 48, 64])
def test_conv_col_f16(gpu, C):
    announce(f"conv col fp16 C={C}")
    rng = np.random.default_rng(200 + C)
    pts, zq_o, nm, zq = _col_setup(gpu)
    M = nm.shape[0]
    x = rng.normal(size=(M, C)).astype(np.float16)
    w = rng.normal(0, 0.05, size=(C, 3, 3, 3, C)).astype(np.float16)
    b = rng.normal(0, 0.05, size=C).astype(np.float32)
    ref = ocv.conv_float(x.astype(np.float64), nm, w.astype(np.float64), dtype=np.float64)
    got = ops.spconv_col(_t(x, gpu), zq, _t(w, gpu), ops.EPI_ACC).cpu().numpy()
    bound = 27 * C * 2 ** -23 * ocv.conv_float(np.abs(x.astype(np.float64)), nm, np.abs(w.astype(np.float64)),
                                                dtype=np.float64)
    assert (np.abs(got - ref) <= bound + 1e-6).all()
    h = ops.spconv_col(_t(x, gpu), zq, _t(w, gpu), ops.EPI_Q, bias=_t(b, gpu)).cpu().numpy()
    _assert_f16_ulp(h, onm.silu_f32((got + b).astype(np.float32)).astype(np.float16))


@pytest.mark.parametrize("prec,C", [("int8", 128), ("fp16", 64), ("fp16", 48)])
def test_conv_col_staged_ragged_tiles(gpu, prec, C):
    """The staged-weight level-0 convolution works on tiles of 8 image rows x 32 columns: a 61 x 83 frame (neither
    a multiple of the tile) in a batch of three, against the dense oracle (int8 bit-exact, fp16 within its
    accumulation bound)."""
    announce(f"conv col staged {prec} C={C} 61x83 x3")
    rng = np.random.default_rng(300 + C)
    pts, zq_o, nm, zq = _col_setup(gpu, H=61, W=83, seed=11, B=3)
    M = nm.shape[0]
    if prec == "int8":
        x = rng.integers(-127, 128, size=(M, C)).astype(np.int8)
        w = rng.integers(-127, 128, size=(C, 3, 3, 3, C)).astype(np.int8)
        acc = ops.spconv_col(_t(x, gpu), zq, _t(w, gpu), ops.EPI_ACC)
        assert np.array_equal(acc.cpu().numpy(), ocv.conv_acc_int(x, nm, w))
    else:
        x = rng.normal(size=(M, C)).astype(np.float16)
        w = rng.normal(0, 0.05, size=(C, 3, 3, 3, C)).astype(np.float16)
        ref = ocv.conv_float(x.astype(np.float64), nm, w.astype(np.float64), dtype=np.float64)
        got = ops.spconv_col(_t(x, gpu), zq, _t(w, gpu), ops.EPI_ACC).cpu().numpy()
        bound = 27 * C * 2 ** -23 * ocv.conv_float(np.abs(x.astype(np.float64)), nm, np.abs(w.astype(np.float64)),
                                                    dtype=np.float64)
        assert (np.abs(got - ref) <= bound + 1e-6).all()
    assert (nm >= 0).sum(1).mean() > 1.5  # the scene has neighbours, not only centre taps


def test_post_depth_after_final_fit(gpu):
    """post_depth (MetricFit.metal:200-211) on the device's final fit: bit-exact against the oracle given the same
    (s, t), +inf off the mask; and the fused step's post_depth option writes the same map."""
    from oracle.fit import post_depth as o_post_depth
    from promptmoge_amd.refiner import RefinerStep

    announce("post_depth after the final fit, config B")
    cfg, sc = _scene("B")
    pts = np.stack([sc.points, sc.points * np.float32(1.01)])
    lid, cnf = np.stack([sc.lidar, sc.lidar]), np.stack([sc.conf, sc.conf])
    mask = np.random.default_rng(3).random(pts.shape[:3]) < 0.9
    P = _t(pts, gpu)
    s, t = ops.fit_final(P, _t(lid, gpu), _t(cnf, gpu), iters=10)
    st = torch.stack([s, t], 1)
    d = ops.post_depth(P, st, _t(mask, gpu)).cpu().numpy()
    st_h = st.cpu().numpy()
    ref = o_post_depth(pts, (st_h[:, 0], st_h[:, 1]), mask)
    assert np.array_equal(d, ref) and np.isinf(d[~mask]).all()
    w = spec.refiner_for(cfg, sc)
    step = RefinerStep(w, 1, cfg.H, cfg.W, fit_iters=10, final_fit=True, post_depth=True)
    Q = _t(sc.points[None], gpu)
    _, fin = step(Q, _t(sc.lidar[None], gpu), _t(sc.conf[None], gpu))
    fh = fin.cpu().numpy()
    assert np.array_equal(step.depth.cpu().numpy(), o_post_depth(Q.cpu().numpy(), (fh[:, 0], fh[:, 1])))
