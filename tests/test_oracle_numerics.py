"""Pins the oracle's fp32 exp/log/SiLU/quantiser: accuracy against float64 math, special values, and bit equality
with the library's own host evaluation of the same source (pmg_math.h), so the NumPy restatement is the function
the kernels run."""
import ctypes as C

import numpy as np
import pytest

from oracle import numerics as nm


def ulp_err(a32, ref64):
    a = a32.astype(np.float64)
    ulp = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    return np.abs(a - ref64) / ulp


def test_exp_accuracy():
    x = np.linspace(-87.0, 88.7, 2_000_001, dtype=np.float32)
    assert ulp_err(nm.exp_f32(x), np.exp(x.astype(np.float64))).max() <= 2.0


def test_exp_special_values():
    assert nm.exp_f32(np.float32(0.0)) == np.float32(1.0)
    assert nm.exp_f32(np.float32(-100.0)) == 0.0
    assert np.isinf(nm.exp_f32(np.float32(100.0)))
    assert np.isnan(nm.exp_f32(np.float32(np.nan)))
    assert nm.exp_f32(np.float32(np.log(2.0))) == np.float32(2.0)


def test_log_accuracy():
    x = np.logspace(-4, 6, 2_000_001).astype(np.float32)
    assert ulp_err(nm.log_f32(x), np.log(x.astype(np.float64))).max() <= 2.0


def test_log_special_values():
    assert nm.log_f32(np.float32(1.0)) == 0.0
    for k in range(-10, 11):
        assert nm.log_f32(np.float32(2.0) ** k) == np.float32(k * np.log(2.0))


def test_silu_accuracy():
    y = np.linspace(-80, 80, 1_000_001, dtype=np.float32)
    y64 = y.astype(np.float64)
    ref = y64 / (1.0 + np.exp(-y64))
    got = nm.silu_f32(y)
    big = np.abs(ref) > 1e-30
    assert (np.abs(got[big] - ref[big]) / np.abs(ref[big])).max() < 4e-7


def test_quant_closed_form():
    mult = np.float32(2.0)
    y = np.array([1.25, 1.75, -1.25, 0.0, 1000.0, -1000.0, 63.25, 63.75], dtype=np.float32)
    # y * 2 = 2.5, 3.5, -2.5, 0, 2000, -2000, 126.5, 127.5 -> half to even, then saturate at +-127
    assert nm.quant_i8(y, mult).tolist() == [2, 4, -2, 0, 127, -127, 126, 127]
    # NaN takes the kernels' clamp (max then min with strict compares): -127; infinities saturate
    assert nm.quant_i8(np.array([np.nan, np.inf, -np.inf], np.float32), mult).tolist() == [-127, 127, -127]


def test_ln_silu_against_float64():
    rng = np.random.default_rng(0)
    x = rng.normal(0.3, 2.0, size=(1000, 48)).astype(np.float32)
    g = (1 + rng.normal(0, 0.1, 48)).astype(np.float32)
    b = rng.normal(0, 0.1, 48).astype(np.float32)
    x64 = x.astype(np.float64)
    y = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-6) * g + b
    ref = y / (1 + np.exp(-y))
    assert np.abs(nm.ln_silu(x, g, b) - ref).max() < 2e-6


@pytest.mark.parametrize("op", [0, 1, 2])
def test_oracle_equals_library_host_math(libpmg, op):
    if op == 1:
        x = np.logspace(-4, 6, 300_001).astype(np.float32)
    else:
        x = np.linspace(-90.0, 90.0, 300_001, dtype=np.float32)
    out = np.empty_like(x)
    assert libpmg.pmg_math_host(op, x.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), x.size) == 0
    ref = [nm.exp_f32, nm.log_f32, nm.silu_f32][op](x)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
