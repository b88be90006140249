"""Pins the oracle's fit_scale_shift restatement: exact-linear recovery, the trimming rule (relative residual with its
1e-3 clamp, the k-th smallest, r <= thr at ties) on hand-built sets whose kept subset is known in closed form,
trimming of outliers above the kept quantile, the < min_points fallback, the degenerate constant-z case, the k
formula, and agreement of the fp64-sum form with the reference's literal fp32 form. A mutation test plants the
plausible misreadings of the rule in the oracle and checks that the hand-built cases catch each of them."""
import numpy as np
import pytest

import fit_cases as fc
from oracle import fit
from oracle.numerics import F32


# The literal fp32 form loses ~1e-5 to the cancellation in n*sxx - sx^2 (the reason the kernel sums in fp64), so its
# bound is looser; shift errors are measured in metres against depths of 0.5-6 m.
@pytest.mark.parametrize("form,tol", [(fit.fit_f64, 2e-6), (fit.fit_f32, 2e-5)])
def test_exact_linear(form, tol):
    rng = np.random.default_rng(0)
    z = rng.uniform(0.5, 6.0, size=(1, 5000)).astype(np.float32)
    t = (1.25 * z.astype(np.float64) + 0.1).astype(np.float32)
    s_, t_ = form(z, t, np.ones_like(z, bool), iters=10)
    assert abs(s_[0] - 1.25) < tol and abs(t_[0] - 0.1) < 2.5 * tol


def test_hand_sized_trim():
    # 40 points on t = 2z + 1, four gross outliers; k = max(int(0.8f * 40), 32) = 32. The first solve sees the
    # outliers; the first trim keeps the 32 smallest residuals, none of them an outlier; the second solve is exact.
    z = np.arange(1, 41, dtype=np.float32)[None]
    t = 2 * z + 1
    t[0, [3, 11, 25, 37]] *= 5.0
    s_, t_, info = fit.fit_f64(z, t, np.ones_like(z, bool), iters=1, return_info=True)
    assert info[0]["k"] == 32 and info[0]["count"] == 40
    assert s_[0] == np.float32(2.0) and abs(t_[0] - 1.0) < 1e-5


def test_outliers_trimmed():
    rng = np.random.default_rng(1)
    z = rng.uniform(0.5, 6.0, size=(1, 20000)).astype(np.float32)
    t = (1.3 * z + 0.05).astype(np.float32)
    bad = rng.random(z.shape) < 0.1
    t = np.where(bad, t * 3.0, t).astype(np.float32)
    s_, t_ = fit.fit_f64(z, t, np.ones_like(z, bool), iters=4)
    assert abs(s_[0] - 1.3) < 1e-5 and abs(t_[0] - 0.05) < 5e-5


def test_too_few_points_returns_identity():
    z = np.ones((2, 100), np.float32) * 3
    t = z * 2
    m = np.zeros_like(z, bool)
    m[0, :31] = True  # 31 < 32
    s_, t_ = fit.fit_f64(z, t, m, iters=4)
    assert s_.tolist() == [1.0, 1.0] and t_.tolist() == [0.0, 0.0]


def test_constant_z():
    rng = np.random.default_rng(2)
    z = np.full((1, 500), 2.0, np.float32)
    t = rng.uniform(1, 3, size=(1, 500)).astype(np.float32)
    s_, t_ = fit.fit_f64(z, t, np.ones_like(z, bool), iters=0)
    assert s_[0] == 1.0 and abs(t_[0] - (t.astype(np.float64).mean() - 2.0)) < 1e-6


def test_k_formula():
    for count, k in [(33, 32), (40, 32), (41, 32), (100, 80), (215040, 172032), (1000001, 800000)]:
        z = np.ones((1, count), np.float32)
        _, _, info = fit.fit_f64(z, z, np.ones_like(z, bool), iters=0, return_info=True)
        assert info[0]["k"] == max(int(np.float32(0.8) * np.float32(count)), 32) == k


def test_fp64_and_fp32_forms_agree_on_a_scene():
    from promptmoge_amd import spec

    cfg = spec.StepConfig("t", 120, 160, 130.0, 130.0, 80.0, 60.0, 16, 1, "int8", seed=3)
    sc = spec.make_scene(cfg)
    z, tg, m, _, _ = fit.prompt_inputs(sc.points[None], sc.lidar[None], sc.conf[None])
    a = fit.fit_f64(z, tg, m, iters=10)
    b = fit.fit_f32(z, tg, m, iters=10)
    assert abs(a[0][0] - b[0][0]) / abs(a[0][0]) < 1e-5 and abs(a[1][0] - b[1][0]) < 1e-5 * max(1, abs(a[1][0]))
    assert abs(a[0][0] - spec.S0) < 0.01  # the generator's affine frame is recovered


@pytest.mark.parametrize("H,W,dh,dw", [(480, 640, 192, 256), (48, 64, 48, 64), (75, 100, 24, 32), (37, 53, 10, 7),
                                       (30, 30, 7, 11), (10, 10, 20, 20)])
def test_area_pool_matches_torch_area_interpolate(H, W, dh, dw):
    """area_pool is F.interpolate(mode='area') bit for bit (window sum in fp32, / height / width)."""
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    x = np.random.default_rng(H * W + dh).uniform(0.3, 7.0, (2, H, W)).astype(np.float32)
    ref = F.interpolate(torch.from_numpy(x)[:, None], (dh, dw), mode="area")[:, 0].numpy()
    assert np.array_equal(fit.area_pool(x, dh, dw).view(np.uint32), ref.view(np.uint32))


def test_final_inputs_mask_rules():
    """v3.py:770-773: conf >= 2, lidar > 0, pooled depth > 0, and (if given) pooled mask_binary > 0.99."""
    H, W = 6, 6
    logz = np.zeros((1, H, W), np.float32)          # depth 1 everywhere
    pts = np.stack([logz, logz, logz], -1)
    lidar = np.array([[[1.0, 0.0], [2.0, np.nan]]], np.float32)
    conf = np.array([[[2.0, 2.0], [1.0, 2.0]]], np.float32)
    z, tg, m = fit.final_inputs(pts, lidar, conf)
    assert np.array_equal(z, np.ones((1, 4), np.float32)) and m.tolist() == [[True, False, False, False]]
    mb = np.ones((1, H, W), bool)
    mb[0, 0, 0] = False                              # 8/9 of the first 3x3 window: 0.889 <= 0.99
    assert fit.final_inputs(pts, lidar, conf, mb)[2].tolist() == [[False, False, False, False]]


def test_post_depth_closed_forms():
    """post_depth (MetricFit.metal:200-211): s = 1, t = 0 gives exp(logz); a shift that makes the depth <= 0 and a
    false mask give +inf; two frames use their own (s, t)."""
    from oracle.fit import post_depth
    from oracle.numerics import exp_f32

    rng = np.random.default_rng(0)
    pts = rng.normal(0, 0.5, (2, 5, 7, 3)).astype(np.float32)
    d = post_depth(pts, ([1.0, 2.0], [0.0, -1.0]))
    assert np.array_equal(d[0], exp_f32(pts[0, ..., 2]))
    e = np.float32(2.0) * exp_f32(pts[1, ..., 2]) - np.float32(1.0)
    assert np.array_equal(d[1], np.where(e > 0, e, np.inf).astype(np.float32))
    assert np.isinf(d[1]).any() and np.isfinite(d[1]).any()
    mask = rng.random((2, 5, 7)) < 0.5
    dm = post_depth(pts, ([1.0, 2.0], [0.0, -1.0]), mask)
    assert np.isinf(dm[~mask]).all() and np.array_equal(dm[mask], d[mask])


# ----------------------------------------------------------------------------- the trimming rule, prompt_stem.py:233-239
FORMS = [(fit.fit_f64, 2e-6), (fit.fit_f32, 2e-6)]


def _solve(form, z, tg, iters=1):
    s_, t_, info = form(z[None], tg[None], np.ones((1, z.size), bool), iters=iters, return_info=True)
    return float(s_[0]), float(t_[0]), info[0]


@pytest.mark.parametrize("form,tol", FORMS)
def test_trim_keeps_the_kth_relative_residual(form, tol):
    """relative_rule_case: the first trim keeps the 31 inliers and Q+; the result is their least-squares line, which
    is 6e-3 away from the line 2z + 0.25 that an absolute residual, a residual over z, the (k+1)-th, or r < thr
    would give."""
    z, tg, kept, line = fc.relative_rule_case()
    s_, t_, info = _solve(form, z, tg)
    es, et = fc.lstsq_st(z, tg, kept)
    assert info["k"] == 32 and len(kept) == 32
    assert abs(s_ - es) < tol and abs(t_ - et) < tol
    assert abs(es - line[0]) > 5e-3 and abs(et - line[1]) > 5e-4      # the misreadings' answer is far away


@pytest.mark.parametrize("form,tol", FORMS)
def test_trim_denominator_is_clamped_at_1e_3(form, tol):
    """clamp_case: a target of 3 * 2^-12 < 1e-3 is divided by 1e-3, which ranks it before the pair point at z = 2;
    without the clamp the other point is kept and the line moves by 5e-3 in s and 0.027 in t."""
    z, tg, kept, wrong = fc.clamp_case()
    s_, t_, _ = _solve(form, z, tg)
    es, et = fc.lstsq_st(z, tg, kept)
    ws, wt = fc.lstsq_st(z, tg, wrong)
    assert abs(s_ - es) < tol and abs(t_ - et) < tol
    assert abs(ws - es) > 1e-3 and abs(wt - et) > 1e-2


@pytest.mark.parametrize("form,tol", FORMS)
def test_trim_keeps_every_tie_at_the_threshold(form, tol):
    """ties_case: the k-th residual is shared by two identical points; r <= thr keeps both (k + 1 points)."""
    z, tg, kept = fc.ties_case()
    s_, t_, info = _solve(form, z, tg)
    es, et = fc.lstsq_st(z, tg, kept)
    assert info["k"] == 36 and len(kept) == 37
    assert abs(s_ - es) < tol and abs(t_ - et) < tol
    assert abs(es - 2.0) > 1e-3


def _pins_hold():
    try:
        for form, tol in FORMS:
            test_trim_keeps_the_kth_relative_residual(form, tol)
            test_trim_denominator_is_clamped_at_1e_3(form, tol)
            test_trim_keeps_every_tie_at_the_threshold(form, tol)
    except AssertionError:
        return False
    return True


def _resid_absolute(s, t, z, tg, mask):
    e = np.abs(np.float32(s) * z + np.float32(t) - tg)
    return np.where(mask, e, F32(np.inf)).astype(np.float32)


def _resid_over_z(s, t, z, tg, mask):
    e = np.abs(np.float32(s) * z + np.float32(t) - tg) / np.maximum(z, F32(1e-3))
    return np.where(mask, e, F32(np.inf)).astype(np.float32)


def _resid_unclamped(s, t, z, tg, mask):
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.abs(np.float32(s) * z + np.float32(t) - tg) / tg
    return np.where(mask, e, F32(np.inf)).astype(np.float32)


def _resid_clamp_1e_4(s, t, z, tg, mask):
    e = np.abs(np.float32(s) * z + np.float32(t) - tg) / np.maximum(tg, F32(1e-4))
    return np.where(mask, e, F32(np.inf)).astype(np.float32)


MUTATIONS = {
    "absolute residual": ("_resid", _resid_absolute),
    "residual over z": ("_resid", _resid_over_z),
    "no 1e-3 clamp": ("_resid", _resid_unclamped),
    "clamp at 1e-4": ("_resid", _resid_clamp_1e_4),
    "k-th one late": ("_kth", lambda r, kk: np.partition(r, kk)[kk]),
    "k-th one early": ("_kth", lambda r, kk: np.partition(r, kk - 2)[kk - 2]),
    "r < thr": ("_keep", lambda mask, r, thr: mask & (r < thr)),
}


def test_pins_hold_on_the_oracle():
    assert _pins_hold()


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_each_misreading_of_the_trim_fails_a_pin(monkeypatch, name):
    """Plants one misreading of prompt_stem.py:233-239 in the CPU oracle; the hand-built cases must reject it."""
    attr, fn = MUTATIONS[name]
    monkeypatch.setattr(fit, attr, fn)
    assert not _pins_hold(), f"the pins do not detect: {name}"
