"""ctypes binding of libpmg.so (the C ABI declared in include/pmg.h).

The library is built in-tree by `python -m promptmoge_amd.build`. There is no fallback: if it is missing or cannot
be loaded, every operation raises, so a GPU run can never silently take another path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libpmg.so")

PMG_OK, PMG_E_INVALID, PMG_E_HIP, PMG_E_OVERFLOW, PMG_E_DEVICE = 0, 1, 2, 3, 4
EPI_ACC, EPI_Q, EPI_R, EPI_BIAS, EPI_SILU, EPI_RLN, EPI_ROUT, EPI_QLIN = 0, 1, 2, 3, 4, 5, 6, 7
PREC_INT8, PREC_FP16 = 0, 1

vp, i32, i64, f32, sz = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t


class PmgError(RuntimeError):
    """A libpmg call returned an error status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"libpmg error {code}: {msg}")
        self.code = code


class ConvEpilogue(C.Structure):
    _fields_ = [
        ("a_scale", f32), ("w_scale", vp), ("bias", vp), ("out_mult", f32), ("skip", vp), ("out", vp),
        ("ln_gamma", vp), ("ln_beta", vp), ("ln_eps", f32), ("next_mult", f32), ("next_q", vp),
        ("out_w", vp), ("out_b", vp), ("points", vp), ("points_out", vp),
    ]


class RefinerConfig(C.Structure):
    _fields_ = [
        ("B", i32), ("H", i32), ("W", i32), ("C", i32), ("n_blocks", i32), ("precision", i32),
        ("depth_resolution", f32), ("dh", i32), ("dw", i32), ("fit_iters", i32), ("fit_trim", f32),
        ("fit_min_points", i32), ("use_prompt", i32), ("soft_gate", i32), ("final_fit", i32), ("use_graph", i32),
        ("output_gate", i32), ("output_gate_floor", f32), ("anchor", f32),
    ]


class BlockWeights(C.Structure):
    _fields_ = [
        ("ln_gamma", vp), ("ln_beta", vp), ("w1", vp), ("w1_scale", vp), ("b1", vp), ("a1_scale", f32),
        ("q1_mult", f32), ("w2", vp), ("w2_scale", vp), ("b2", vp), ("a2_scale", f32), ("q2_mult", f32),
    ]


class UNetConfig(C.Structure):
    _fields_ = [
        ("B", i32), ("H", i32), ("W", i32), ("levels", i32), ("channels", i32 * 8), ("enc_blocks", i32 * 8),
        ("dec_blocks", i32 * 8), ("bottleneck_blocks", i32), ("enc_channels", i32), ("depth_resolution", f32),
        ("use_graph", i32), ("precision", i32),
    ]


class UNetStepConfig(C.Structure):
    _fields_ = [
        ("dh", i32), ("dw", i32), ("fit_iters", i32), ("fit_trim", f32), ("fit_min_points", i32),
        ("use_prompt", i32), ("soft_gate", i32), ("output_gate", i32), ("output_gate_floor", f32), ("anchor", f32),
        ("final_fit", i32),
    ]


class LinearWeights(C.Structure):
    _fields_ = [("w", vp), ("w_scale", vp), ("bias", vp), ("a_scale", f32), ("q_mult", f32)]


class RefinerWeights(C.Structure):
    _fields_ = [
        ("in_w", vp), ("in_b", vp), ("pr_w", vp), ("pr_b", vp), ("out_w", vp), ("out_b", vp),
        ("n_blocks", i32), ("blocks", C.POINTER(BlockWeights)),
    ]


class UNetWeights(C.Structure):
    _fields_ = [
        ("in_w", vp), ("in_b", vp), ("pr_w", vp), ("pr_b", vp), ("out_w", vp), ("out_b", vp),
        ("n_blocks", i32), ("blocks", C.POINTER(BlockWeights)), ("n_linears", i32),
        ("linears", C.POINTER(LinearWeights)),
    ]


UNET_COUNTS, UNET_COORDS, UNET_PARENT, UNET_NMAP, UNET_TILE_MASK, UNET_DOWN, UNET_UP, UNET_ENC_TOKENS, \
    UNET_COL_OFFSETS, UNET_STEP_ST = range(10)

# name -> (restype, argtypes)
SIGNATURES = {
    "pmg_last_error": (C.c_char_p, []),
    "pmg_version": (i32, []),
    "pmg_math_host": (i32, [i32, vp, vp, i64]),
    "pmg_math_device": (i32, [i32, vp, vp, i64, vp]),
    "pmg_probe_copy": (i32, [vp, vp, i64, vp]),
    "pmg_probe_mfma_i8": (i32, [i32, i32, vp, vp]),
    "pmg_voxelize": (i32, [vp, i64, i32, i32, i32, f32, vp, vp, vp, vp]),
    "pmg_nmap_column": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp, vp]),
    "pmg_hash_workspace_bytes": (sz, [i64]),
    "pmg_nmap_hash": (i32, [vp, i64, vp, vp, vp, vp, vp, vp, sz, vp]),
    "pmg_sorted_workspace_bytes": (sz, [vp]),
    "pmg_nmap_sorted": (i32, [vp, i64, vp, vp, vp, vp, vp, vp, sz, vp]),
    "pmg_pool_cache_workspace_bytes": (sz, [i64]),
    "pmg_pool_cache": (i32, [vp, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]),
    "pmg_sparse_pool": (i32, [vp, i64, i32, vp, vp, i64, i32, vp, vp]),
    "pmg_sparse_upsample": (i32, [vp, i64, vp, i64, vp, vp]),
    "pmg_row_order_workspace_bytes": (sz, [i64]),
    "pmg_row_order": (i32, [vp, vp, i64, i64, vp, vp, vp, vp, sz, vp]),
    "pmg_nmap_from_rows": (i32, [vp, i64, vp, vp, vp]),
    "pmg_kmap_workspace_bytes": (sz, [i64]),
    "pmg_kmap_compact": (i32, [vp, i64, vp, vp, vp, i64, vp, sz, vp]),
    "pmg_spconv_i8": (i32, [vp, vp, vp, i64, i32, i32, vp, i32, f32, vp, vp, f32, vp, vp, vp]),
    "pmg_spconv_i8_ordered": (i32, [vp, vp, vp, vp, i64, i32, i32, vp, i32, f32, vp, vp, f32, vp, vp, vp]),
    "pmg_spconv_f16": (i32, [vp, vp, vp, i64, i32, i32, vp, i32, vp, vp, vp, vp]),
    "pmg_spconv_bf16": (i32, [vp, vp, vp, i64, i32, i32, vp, i32, vp, vp, vp, vp]),
    "pmg_spconv_f32": (i32, [vp, vp, vp, i64, i32, i32, vp, i32, vp, vp, vp]),
    "pmg_spconv_col": (i32, [i32, vp, vp, i32, i32, i32, i32, vp, i32, C.c_void_p, vp]),
    "pmg_ln_silu_quant": (i32, [vp, i64, i32, vp, vp, f32, f32, vp, vp]),
    "pmg_ln_silu_f16": (i32, [vp, i64, i32, vp, vp, f32, vp, vp]),
    "pmg_fit_workspace_bytes": (sz, [i64, i32]),
    "pmg_debug_fit_spin_limit": (C.c_uint, [C.c_uint]),
    "pmg_debug_fit_plan": (C.c_uint, [C.c_uint]),
    "pmg_fit_scale_shift_static": (i32, [vp, vp, vp, i32, i64, i32, f32, i32, vp, vp, vp]),
    "pmg_fit_scale_shift": (i32, [vp, vp, vp, i32, i64, i32, f32, i32, vp, vp, vp, sz, vp]),
    "pmg_fit_prompt": (i32, [vp, i64, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, vp, vp, vp, sz, vp]),
    "pmg_fit_final_workspace_bytes": (sz, [i32, i32, i32, i32]),
    "pmg_post_depth": (i32, [vp, i64, vp, i32, i32, i32, vp, vp, vp]),
    "pmg_fit_final": (i32, [vp, i64, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, vp, vp, vp, sz, vp]),
    "pmg_nearest_fill_workspace_bytes": (sz, [i32, i32, i32]),
    "pmg_nearest_fill": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp, sz, vp]),
    "pmg_gauge_poly_workspace_bytes": (sz, [i32, i32, i32]),
    "pmg_gauge_poly": (i32, [vp, i32, i32, i32, vp, vp, i32, i32, i32, i32, vp, vp, vp, sz, vp]),
    "pmg_refiner_create": (vp, [C.POINTER(RefinerConfig)]),
    "pmg_refiner_destroy": (None, [vp]),
    "pmg_refiner_set_weights": (i32, [vp, C.POINTER(RefinerWeights)]),
    "pmg_refiner_step": (i32, [vp, vp, vp, vp, vp, vp, vp, vp]),
    "pmg_refiner_forward": (i32, [vp, vp, vp, vp, vp, vp]),
    "pmg_refiner_check": (i32, [vp, vp]),
    "pmg_refiner_buffer": (vp, [vp, i32]),
    "pmg_unet_create": (vp, [C.POINTER(UNetConfig)]),
    "pmg_unet_destroy": (None, [vp]),
    "pmg_unet_workspace_bytes": (sz, [vp]),
    "pmg_unet_capacity": (i64, [vp]),
    "pmg_unet_set_weights": (i32, [vp, C.POINTER(UNetWeights)]),
    "pmg_unet_forward": (i32, [vp, vp, vp, vp, vp, vp, vp, vp]),
    "pmg_unet_buffer": (vp, [vp, i32, i32]),
    "pmg_unet_step_prepare": (i32, [vp, C.POINTER(UNetStepConfig)]),
    "pmg_unet_step": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
    "pmg_unet_check": (i32, [vp, vp]),
}

_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """Loads libpmg.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built; run `python -m promptmoge_amd.build`")
        h = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def check(code: int) -> None:
    if code != PMG_OK:
        raise PmgError(code, lib().pmg_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
