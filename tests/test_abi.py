"""The C ABI without a GPU: the library loads, exports every function include/pmg.h declares (with the argument
count the binding uses), and rejects invalid arguments on the host before any launch."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from promptmoge_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "pmg.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(pmg_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S)
    out = {}
    for name, args in decls:
        args = " ".join(args.split())
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_header_parsed():
    fns = declared_functions()
    assert "pmg_refiner_step" in fns and "pmg_spconv_i8" in fns and len(fns) >= 20


def test_every_declared_symbol_is_exported_and_bound(libpmg):
    fns = declared_functions()
    for name, nargs in fns.items():
        assert hasattr(libpmg, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes binding"
        assert len(_lib.SIGNATURES[name][1]) == nargs, f"{name}: binding has {len(_lib.SIGNATURES[name][1])} args, header {nargs}"
    assert set(_lib.SIGNATURES) == set(fns)


def test_version_and_error_string(libpmg):
    assert libpmg.pmg_version() == 5
    rc = libpmg.pmg_voxelize(None, 1, 1, 1, 1, 256.0, None, None, None, None)
    assert rc == _lib.PMG_E_INVALID
    assert b"null" in libpmg.pmg_last_error()


def test_invalid_shapes_rejected_on_host(libpmg):
    dummy = C.c_void_p(16)  # never dereferenced: validation fails first
    # Co not a multiple of 16
    assert libpmg.pmg_spconv_i8(dummy, dummy, dummy, 10, 16, 24, dummy, 0, 1.0, dummy, None, 1.0, None, dummy,
                                None) == _lib.PMG_E_INVALID
    # Ci*1 not a multiple of 16
    assert libpmg.pmg_spconv_i8(dummy, dummy, dummy, 10, 24, 32, dummy, 0, 1.0, dummy, None, 1.0, None, dummy,
                                None) == _lib.PMG_E_INVALID
    # fp32 conv with a Q epilogue
    assert libpmg.pmg_spconv_f32(dummy, dummy, dummy, 10, 16, 16, dummy, 1, None, dummy, None) == _lib.PMG_E_INVALID
    # unsupported LayerNorm width
    assert libpmg.pmg_ln_silu_quant(dummy, 10, 40, dummy, dummy, 1e-6, 1.0, dummy, None) == _lib.PMG_E_INVALID
    # fit: N out of range, workspace too small, min_points < 1
    assert libpmg.pmg_fit_scale_shift(dummy, dummy, dummy, 1, 0, 4, 0.2, 32, dummy, None, dummy, 1 << 20,
                                      None) == _lib.PMG_E_INVALID
    assert libpmg.pmg_fit_scale_shift(dummy, dummy, dummy, 1, 1000, 4, 0.2, 32, dummy, None, dummy, 16,
                                      None) == _lib.PMG_E_INVALID
    assert libpmg.pmg_fit_scale_shift(dummy, dummy, dummy, 1, 1000, 4, 0.2, 0, dummy, None, dummy, 1 << 20,
                                      None) == _lib.PMG_E_INVALID
    # hash: shape too large for 64-bit keys
    big = (C.c_int64 * 4)(1 << 20, 1 << 20, 1 << 20, 1 << 20)
    assert libpmg.pmg_nmap_hash(C.c_void_p(16), 5, big, None, None, None, None, dummy, 1 << 30,
                                None) == _lib.PMG_E_INVALID
    # sorted map: workspace too small, unaligned workspace, more than 2^31 columns
    sh = (C.c_int64 * 4)(1, 64, 64, 64)
    assert libpmg.pmg_nmap_sorted(C.c_void_p(16), 5, sh, None, None, None, None, C.c_void_p(256), 64,
                                  None) == _lib.PMG_E_INVALID
    assert libpmg.pmg_nmap_sorted(C.c_void_p(16), 5, sh, None, None, None, None, C.c_void_p(260), 1 << 20,
                                  None) == _lib.PMG_E_INVALID
    wide = (C.c_int64 * 4)(4, 1 << 16, 1 << 16, 8)
    assert libpmg.pmg_nmap_sorted(C.c_void_p(16), 5, wide, None, None, None, None, C.c_void_p(256), 1 << 40,
                                  None) == _lib.PMG_E_INVALID
    # ordered conv: only Ci = Co = 64 / 128
    assert libpmg.pmg_spconv_i8_ordered(dummy, dummy, dummy, dummy, 10, 32, 32, dummy, 0, 1.0, dummy, None, 1.0,
                                        None, dummy, None) == _lib.PMG_E_INVALID


def test_refiner_create_rejects_bad_config(libpmg):
    cfg = _lib.RefinerConfig(1, 8, 8, 40, 1, 0, 256.0, 8, 8, 4, 0.2, 32, 1, 0, 0, 1)  # C=40 unsupported
    assert not libpmg.pmg_refiner_create(C.byref(cfg))
    assert b"unsupported" in libpmg.pmg_last_error()


def test_workspace_sizes(libpmg):
    assert libpmg.pmg_hash_workspace_bytes(1_000_000) >= 4 * 1_000_000 * 12
    # sorted map: a status line plus a (start, end) run per (b, x, y) column; 0 beyond 2^31 columns
    assert libpmg.pmg_sorted_workspace_bytes((C.c_int64 * 4)(2, 1024, 1024, 1024)) == 256 + 8 * 2 * 1024 * 1024
    assert libpmg.pmg_sorted_workspace_bytes((C.c_int64 * 4)(4, 1 << 16, 1 << 16, 8)) == 0
    assert libpmg.pmg_fit_workspace_bytes(307_200, 10) >= 10 * 3 * 2048 * 4
    assert libpmg.pmg_kmap_workspace_bytes(1000) >= 27 * 4 * 4


def test_nearest_fill_rejected_on_host(libpmg):
    dummy = C.c_void_p(16)
    ws = libpmg.pmg_nearest_fill_workspace_bytes(1, 8, 8)
    assert ws >= 8 * 8 * 4
    # map taller than the LDS column buffer
    assert libpmg.pmg_nearest_fill(dummy, None, 1, 8193, 8, dummy, None, None, dummy, 1 << 30,
                                   None) == _lib.PMG_E_INVALID
    # conf without conf_out
    assert libpmg.pmg_nearest_fill(dummy, dummy, 1, 8, 8, dummy, None, None, dummy, ws, None) == _lib.PMG_E_INVALID
    # workspace too small
    assert libpmg.pmg_nearest_fill(dummy, None, 1, 8, 8, dummy, None, None, dummy, ws - 1,
                                   None) == _lib.PMG_E_INVALID


def test_gauge_rejected_on_host(libpmg):
    dummy = C.c_void_p(16)
    ws = libpmg.pmg_gauge_poly_workspace_bytes(2, 24, 32)
    assert ws >= 2 * 24 * 32 * 13
    assert libpmg.pmg_gauge_poly_workspace_bytes(0, 24, 32) == 0
    args = lambda **k: dict(dict(depth=dummy, B=2, H=48, W=64, lidar=dummy, conf=None, h=24, w=32, degree=2, iters=3,
                                 corr=dummy, coef=dummy, ws=dummy, wsb=ws), **k)
    call = lambda a: libpmg.pmg_gauge_poly(a["depth"], a["B"], a["H"], a["W"], a["lidar"], a["conf"], a["h"], a["w"],
                                           a["degree"], a["iters"], a["corr"], a["coef"], a["ws"], a["wsb"], None)
    assert call(args(degree=0)) == _lib.PMG_E_INVALID           # degree must be >= 1
    assert call(args(iters=0)) == _lib.PMG_E_INVALID            # the reference needs one lstsq round
    assert call(args(wsb=ws - 1)) == _lib.PMG_E_INVALID         # workspace too small
    assert call(args(corr=None)) == _lib.PMG_E_INVALID          # null output
    assert call(args(h=0)) == _lib.PMG_E_INVALID


def test_refiner_create_rejects_bad_gate_and_anchor(libpmg):
    base = (1, 8, 8, 32, 1, 0, 256.0, 8, 8, 4, 0.2, 32, 1, 0, 0, 1)
    for extra in [(1, 1.5, 0.0), (1, -0.1, 0.0), (0, 0.1, 1.5), (0, 0.1, -0.5)]:
        cfg = _lib.RefinerConfig(*base, *extra)
        assert not libpmg.pmg_refiner_create(C.byref(cfg))
        assert b"unsupported" in libpmg.pmg_last_error()


def test_python_ops_refuse_host_tensors():
    import torch

    from promptmoge_amd import ops

    with pytest.raises(ValueError, match="GPU tensor"):
        ops.gauge_poly(torch.ones(1, 8, 8), torch.ones(1, 4, 4))


def test_header_compiles_as_plain_c(tmp_path):
    """include/pmg.h is the C ABI a non-Python binding includes: it must compile as C99 with no C++ in it."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "use_pmg.c"
    src.write_text('#include "pmg.h"\nint main(void) { return pmg_version() == 0; }\n')
    inc = Path(__file__).resolve().parents[1] / "include"
    r = subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", f"-I{inc}", str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_refiner_create_rejects_maps_beyond_the_fit(libpmg):
    """The metric fit holds 2^21 elements per batch item: a prompt fit (or anchor re-fit) over a larger H x W map,
    or a final fit over a larger LiDAR grid, is refused when the context is created, not at every step."""
    big = (1 << 21) + 2048  # 1025 x 2048 pixels
    # (B, H, W, C, n_blocks, prec, res, dh, dw, iters, trim, min_points, use_prompt, soft, final_fit, graph)
    cfg = _lib.RefinerConfig(1, 1025, 2048, 32, 1, 0, 256.0, 8, 8, 4, 0.2, 32, 1, 0, 0, 1)
    assert big == 1025 * 2048
    assert not libpmg.pmg_refiner_create(C.byref(cfg))
    assert b"exceeds the metric fit" in libpmg.pmg_last_error() and b"use_prompt" in libpmg.pmg_last_error()
    cfg = _lib.RefinerConfig(1, 1025, 2048, 32, 1, 0, 256.0, 8, 8, 4, 0.2, 32, 0, 0, 0, 1, 0, 0.1, 0.5)
    assert not libpmg.pmg_refiner_create(C.byref(cfg))
    assert b"anchor" in libpmg.pmg_last_error()
    cfg = _lib.RefinerConfig(1, 64, 64, 32, 1, 0, 256.0, 1025, 2048, 4, 0.2, 32, 0, 0, 1, 1)
    assert not libpmg.pmg_refiner_create(C.byref(cfg))
    assert b"final_fit" in libpmg.pmg_last_error()


def test_fit_plan_hook_round_trips(libpmg):
    prev = libpmg.pmg_debug_fit_plan(2)
    assert prev == 0
    assert libpmg.pmg_debug_fit_plan(9) == 2  # out of range: the normal plan
    assert libpmg.pmg_debug_fit_plan(0) == 0


def test_fit_spin_limit_hook_round_trips(libpmg):
    prev = libpmg.pmg_debug_fit_spin_limit(7)
    assert prev == 1 << 23
    assert libpmg.pmg_debug_fit_spin_limit(0) == 7
    assert libpmg.pmg_debug_fit_spin_limit(0) == 1 << 23


def test_unet_create_rejects_bad_config(libpmg):
    """pmg_unet_create validates on the host, before any allocation (sparse_unet.py:52, 187 and the kernels'
    widths)."""
    def cfg(**kw):
        d = dict(B=1, H=64, W=96, levels=3, channels=[16, 32, 32], enc_blocks=[1, 1, 1], dec_blocks=[1, 1], bott=1,
                 enc=32)
        d.update(kw)
        pad = lambda xs: (C.c_int * 8)(*(list(xs) + [0] * (8 - len(xs))))
        return _lib.UNetConfig(d["B"], d["H"], d["W"], d["levels"], pad(d["channels"]), pad(d["enc_blocks"]),
                               pad(d["dec_blocks"]), d["bott"], d["enc"], 256.0, 1)
    for bad, msg in [(dict(levels=1), b"levels"), (dict(H=62), b"multiples"), (dict(channels=[24, 32, 32]), b"level-0"),
                     (dict(channels=[16, 40, 32]), b"widths"), (dict(dec_blocks=[1, 0]), b"last up stage"),
                     (dict(enc=20), b"enc_channels")]:
        c = cfg(**bad)
        assert not libpmg.pmg_unet_create(C.byref(c)), bad
        assert msg in libpmg.pmg_last_error(), (bad, libpmg.pmg_last_error())
    assert libpmg.pmg_unet_forward(None, None, None, None, None, None, None, None) == _lib.PMG_E_INVALID
    assert libpmg.pmg_unet_buffer(None, 0, 0) is None and libpmg.pmg_unet_capacity(None) == 0
