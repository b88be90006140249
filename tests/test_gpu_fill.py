"""GPU parity of nearest_fill (promptmoge/model.py:61-72) against the oracle (itself pinned against scipy's EDT):
filled depth, confidence and source index are bit-exact."""
import numpy as np
import pytest
import torch

from oracle import fill as ofill
from promptmoge_amd import ops, prompt

from conftest import announce

pytestmark = pytest.mark.gpu


def _case(rng, h, w, hole, big_hole=False):
    depth = rng.uniform(0.5, 6.0, (h, w)).astype(np.float32)
    depth[rng.random((h, w)) < hole] = 0.0
    if big_hole:
        depth[: h // 5] = 0.0                                   # a band without returns (sky)
        depth[h // 2: h // 2 + h // 4, w // 3: w // 3 + w // 3] = -1.0
    conf = rng.integers(0, 3, (h, w)).astype(np.float32)
    return depth, conf


def _expect(depth, conf):
    valid = depth > 0
    if not valid.any():
        return depth, conf, np.full(depth.shape, -1, np.int64)
    idx = ofill.nearest_index(valid)
    return depth[idx[0], idx[1]], np.where(valid, conf, 1).astype(np.float32), idx[0] * depth.shape[1] + idx[1]


def _check(depth, conf, gpu):
    d, c, i = ops.nearest_fill(torch.from_numpy(depth).to(gpu), torch.from_numpy(conf).to(gpu), return_index=True)
    torch.cuda.synchronize()
    for k in range(depth.shape[0]):
        ed, ec, ei = _expect(depth[k], conf[k])
        np.testing.assert_array_equal(i[k].cpu().numpy(), ei)
        np.testing.assert_array_equal(d[k].cpu().numpy().view(np.uint32), ed.view(np.uint32))
        np.testing.assert_array_equal(c[k].cpu().numpy(), ec)


@pytest.mark.parametrize("h,w,hole", [(1, 1, 0.5), (1, 70, 0.6), (70, 1, 0.6), (5, 64, 0.3), (65, 130, 0.5),
                                      (64, 65, 0.9), (200, 300, 0.2), (37, 500, 0.97)])
def test_fill_random(gpu, h, w, hole):
    announce(f"nearest_fill {h}x{w} hole={hole}")
    rng = np.random.default_rng(h * 1000 + w)
    d, c = _case(rng, h, w, hole)
    _check(d[None], c[None], gpu)


def test_fill_tie_lattices_and_batch(gpu):
    announce("nearest_fill lattices, batch of 5 incl. empty and full images")
    h, w = 61, 77
    rng = np.random.default_rng(11)
    depth = np.zeros((5, h, w), np.float32)
    depth[0, ::3, ::3] = 1.0 + rng.random((21, 26))
    depth[1, ::4, ::7] = 1.0 + rng.random((16, 11))
    depth[2, 0, 0] = depth[2, h - 1, w - 1] = 2.0
    depth[3] = 3.0                                    # all valid: unchanged
    depth[4] = np.where(rng.random((h, w)) < 0.5, -0.0, np.nan)   # no valid pixel: unchanged
    conf = rng.integers(0, 3, (5, h, w)).astype(np.float32)
    _check(depth, conf, gpu)


def test_fill_config_h_size(gpu):
    announce("nearest_fill 756x1008, 20 % holes + large holes")
    rng = np.random.default_rng(5)
    d, c = _case(rng, 756, 1008, 0.2, big_hole=True)
    _check(d[None], c[None], gpu)


def test_fill_in_place(gpu):
    announce("nearest_fill in place")
    rng = np.random.default_rng(9)
    d, c = _case(rng, 90, 150, 0.4, big_hole=True)
    td, tc = torch.from_numpy(d).to(gpu), torch.from_numpy(c).to(gpu)
    ops.nearest_fill(td, tc, out=(td, tc))
    ed, ec, _ = _expect(d, c)
    np.testing.assert_array_equal(td.cpu().numpy(), ed)
    np.testing.assert_array_equal(tc.cpu().numpy(), ec)


def test_fill_numpy_mirror_keeps_dtypes(gpu):
    announce("prompt.nearest_fill numpy float64 / uint8")
    rng = np.random.default_rng(21)
    d = rng.uniform(0.5, 6.0, (48, 80))
    d[rng.random(d.shape) < 0.35] = 0.0
    d[3, 3] = 1e-300                      # positive in float64, zero in float32: still a valid pixel
    c = rng.integers(0, 3, d.shape).astype(np.uint8)
    got_d, got_c = prompt.nearest_fill(d, c)
    exp_d, exp_c = ofill.nearest_fill(d, c)
    assert got_d.dtype == np.float64 and got_c.dtype == np.uint8
    np.testing.assert_array_equal(got_d, exp_d)
    np.testing.assert_array_equal(got_c, exp_c)
    full = np.ones((4, 4))
    assert prompt.nearest_fill(full, c[:4, :4])[0] is full
