"""Hand-built inputs that pin the trimming rule of fit_scale_shift (moge/model/modules/prompt_stem.py:233-239):

    r = |s*z + t - target| / target.clamp_min(1e-3);  thr = kthvalue(r, k);  w = mask & (r <= thr)

Every case is built so that its FIRST solve is an exact line: besides the inliers (on the line), every other point
comes in a pair at one z with targets L(z) + e and L(z) - e, so the pairs add nothing to the weighted sums beyond
what the line gives. The first residuals are then known in closed form (exactly 0 on the inliers, e / target on a
pair), the first trim keeps a subset that is written out below by hand, and with iters=1 the result is the
least-squares line of that subset (np.polyfit, independent of the oracle). Each case is chosen so that one plausible
misreading of the rule keeps a different subset, whose least-squares line is far from the right one.
"""
from __future__ import annotations

import numpy as np


def _pack(inl, pairs, line):
    """inl: inlier z values; pairs: (z, e) with targets line(z) +- e. Returns z, target (fp32, exact binary
    fractions), and the index of each pair member: {(z, +1): i, (z, -1): i}."""
    s0, t0 = line
    z, tg, where = [], [], {}
    for v in inl:
        z.append(v)
        tg.append(s0 * v + t0)
    for v, e in pairs:
        for sign in (+1, -1):
            where[(v, sign)] = len(z)
            z.append(v)
            tg.append(s0 * v + t0 + sign * e)
    z = np.array(z, np.float64)
    tg = np.array(tg, np.float64)
    assert np.array_equal(z.astype(np.float32).astype(np.float64), z)      # exact in fp32
    assert np.array_equal(tg.astype(np.float32).astype(np.float64), tg)
    return z.astype(np.float32), tg.astype(np.float32), where


def lstsq_st(z, tg, idx):
    """Least-squares (s, t) of the points idx, in float64 by np.polyfit."""
    s, t = np.polyfit(z[idx].astype(np.float64), tg[idx].astype(np.float64), 1)
    return s, t


def relative_rule_case():
    """41 points, k = int(0.8f * 41) = 32 (k-th of the 41 residuals). Line target = 2z + 0.25.

    31 inliers; pair P at z = 0.125 (line 0.5, e = 0.125): relative residuals 0.2 / 0.333, absolute 0.125 / 0.125;
    pair Q at z = 2.875 (line 6, e = 0.5): relative 0.0769 / 0.0909, absolute 0.5 / 0.5; three far pairs (relative
    >= 0.35, absolute >= 2, residual / z >= 1.1).

    The rule keeps the inliers and Q+ (the 32nd smallest relative residual) -> the line of those 32 points.
    Misreadings, each of which keeps a set whose line is exactly 2z + 0.25:
      absolute residual |e|:       the k-th is P's 0.125, tied, both kept (inliers + P+ + P-);
      residual / z:                Q's 0.174 is the smallest, tied, both kept;
      k-th one position late:      the threshold is Q-'s 0.0909 (inliers + Q+ + Q-);
      r < thr instead of r <= thr: only the inliers.
    """
    inl = [0.5 + j / 8 for j in range(31)]
    pairs = [(0.125, 0.125), (2.875, 0.5), (1.0, 2.0), (1.5, 2.5), (3.5, 4.0)]
    z, tg, where = _pack(inl, pairs, (2.0, 0.25))
    kept = list(range(31)) + [where[(2.875, +1)]]
    return z, tg, kept, (2.0, 0.25)


def clamp_case():
    """41 points, k = 32. Line target = z.

    29 inliers; pair X at z = 2^-10 with e = 2^-12: targets 5 * 2^-12 (above 1e-3) and 3 * 2^-12 (below 1e-3, so
    the denominator is clamped to 1e-3): relative residuals 0.2 and 0.244 (0.333 without the clamp); pair Y at
    z = 2 (e = 0.4375): 0.179 and 0.28; four far pairs (>= 0.44).

    The rule keeps the inliers, Y+, X+ and X- (the three smallest of the pairs). Without the clamp X- moves to
    0.333, behind Y-'s 0.28, so the inliers, Y+, X+ and Y- are kept instead.
    """
    inl = [1 + j / 8 for j in range(29)]
    pairs = [(2.0 ** -10, 2.0 ** -12), (2.0, 0.4375), (3.0, 2.5), (4.0, 3.0), (1.5, 1.25), (2.5, 2.0)]
    z, tg, where = _pack(inl, pairs, (1.0, 0.0))
    kept = list(range(29)) + [where[(2.0, +1)], where[(2.0 ** -10, +1)], where[(2.0 ** -10, -1)]]
    wrong = list(range(29)) + [where[(2.0, +1)], where[(2.0 ** -10, +1)], where[(2.0, -1)]]
    return z, tg, kept, wrong


def ties_case():
    """45 points, k = int(0.8f * 45) = 36. Line target = 2z + 0.25.

    35 inliers; pair Q (z = 2.875, e = 0.5) twice, so two identical Q+ points and two identical Q- points; three far
    pairs. The 36th and 37th smallest residuals are the two Q+ copies: the threshold equals both, and r <= thr keeps
    37 points, one more than k (r < thr would keep only the 35 inliers)."""
    inl = [0.5 + j / 8 for j in range(35)]
    pairs = [(2.875, 0.5), (2.875, 0.5), (1.0, 2.0), (1.5, 2.5), (3.5, 4.0)]
    z, tg, _ = _pack(inl, pairs, (2.0, 0.25))
    kept = list(range(35)) + [35, 37]          # the two Q+ copies (each pair is stored as +, -)
    assert tg[35] == tg[37] == 6.5
    return z, tg, kept
