"""The refiner's layers, restated from the reference (test infrastructure only): the int8 contract, the residual
block and the linear layers, shared by the single-level step (oracle/refiner.py) and the U-Net (oracle/unet.py).

Arithmetics ("mode"):
  "fp32"       the reference module in fp32: torch's LayerNorm (eps 1e-6), SiLU x / (1 + exp(-x)), nn.Linear, and
               _fallback's fp32 submanifold conv (bias first, taps ascending; _core.py:399-441)
  "fakequant"  the module under enable_refiner_qat (qat.py:118-138): the input of every quantised layer fake-quantised
               per tensor with scale clip/127 (qat.py:28-37, 89-98), its weight per output channel (qat.py:40-57)
  "int8"       the deployed integer arithmetic (SparseConvInt8.metal:1-154, Refiner.metal:75-131, 133-322): int8 codes
               clamp(rint(y * 127/clip)), exact int32 accumulation, (acc * a_scale) * w_scale[n] + bias[n] in fp32,
               LayerNorm in the kernels' fixed "quad" summation order, exp/log/SiLU bit-reproducible (numerics.py)
  "fp16"       the teacher (PromptMoGe-L) in half precision: every conv and linear on fp16 operands (activations and
               weights rounded to fp16) with fp32 accumulation (here fp64, then rounded; `acc=np.float32` sums in
               fp32 instead, another order of the same arithmetic), LayerNorm + SiLU in fp32
               (quad order) rounded to fp16 as conv1's input, SiLU of conv1 rounded to fp16 as conv2's input, the
               residual stream, pooling, upsampling, input_proj and out_proj in fp32 (the single-level teacher's
               contract, refiner.blocks_fp16, extended to the U-Net's linears)
"""
from __future__ import annotations

import numpy as np

from .conv import conv_acc_int, conv_float, dequant, epilogue_q, epilogue_r
from .numerics import F32, ln_silu, quad_sum, quant_i8, rowwise


# ------------------------------------------------------------------------------------------------- int8 contract
def quantize_weight(w):
    """WeightFakeQuant (qat.py:52-57) with _fake_quant (qat.py:35-36): s = max|W[co]| / 127 in fp32, clamped at
    1e-12, q = clamp(round(W / s), -127, 127). A weight stored already quantised (an object with `q` and `s`, as
    refiner.bin holds them, export/refiner.py:40-46) is returned as stored."""
    if hasattr(w, "q") and hasattr(w, "s"):
        return np.asarray(w.q, np.int8), np.asarray(w.s, np.float32)
    w = np.asarray(w, dtype=np.float32)
    s = (np.abs(w).reshape(w.shape[0], -1).max(axis=1) / F32(127.0)).astype(np.float32)
    s = np.maximum(s, F32(1e-12))
    q = np.clip(np.rint(w / s.reshape((-1,) + (1,) * (w.ndim - 1))), -127, 127)
    return q.astype(np.int8), s


def act_scale(clip: float) -> np.float32:
    """ActFakeQuant scale clip / QMAX in fp32, clamped at 1e-12 (qat.py:35, 98); the deployed dequantisation scale
    aScale = clip / 127 (Refiner.swift:147)."""
    return np.maximum(F32(clip) / F32(127.0), F32(1e-12))


def act_mult(clip: float) -> np.float32:
    """The deployed requantisation multiplier 127 / clip in fp32 (Refiner.swift:148)."""
    return F32(127.0) / F32(clip)


def fake_quant(x, clip):
    """_fake_quant's forward value (qat.py:35-36): clamp(round(x / s), -127, 127) * s, s = clip / 127."""
    s = act_scale(clip)
    return (np.clip(np.rint(np.asarray(x, np.float32) / s), -127, 127) * s).astype(np.float32)


def fake_quant_weight(w):
    """WeightFakeQuant's value (qat.py:52-57): q * s per output channel (axis 0)."""
    q, s = quantize_weight(w)
    return (q.astype(np.float32) * s.reshape((-1,) + (1,) * (q.ndim - 1))).astype(np.float32)


def qat_codes(x, clip):
    """The integers the QAT fake quantiser rounds to, clamp(round(x / s), -127, 127) with s = clip / 127 (qat.py:36):
    the division form; the deployed kernels multiply by 127 / clip instead (see quant_i8)."""
    return np.clip(np.rint(np.asarray(x, np.float32) / act_scale(clip)), -127, 127).astype(np.int8)


# ------------------------------------------------------------------------------------------------- torch fp32 ops
def layer_norm(x, gamma, beta, eps=1e-6):
    """nn.LayerNorm(eps=1e-6, affine) in fp32 (flex_sparse_blocks.py:56)."""
    x = np.asarray(x, np.float32)
    mu = x.mean(axis=1, keepdims=True, dtype=np.float32)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True, dtype=np.float32)
    return ((x - mu) / np.sqrt(var + F32(eps)) * gamma + beta).astype(np.float32)


def silu(x):
    """F.silu in fp32."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore"):
        return (x / (F32(1.0) + np.exp(-x))).astype(np.float32)


# ------------------------------------------------------------------------------------------------- layers
def input_proj(f: np.ndarray, w, res=None, gate=None) -> np.ndarray:
    """input_proj (+ prompt_proj) (sparse_unet.py:189-192), in the kernel's order: ((b + w0 f0) + w1 f1) + w2 f2
    (+ ((pb + p0 r) + p1 g))."""
    in_w, in_b = np.asarray(w.in_w, np.float32), np.asarray(w.in_b, np.float32)
    y = in_b[None, :] + in_w[None, :, 0] * f[:, 0:1]
    y = y + in_w[None, :, 1] * f[:, 1:2]
    y = y + in_w[None, :, 2] * f[:, 2:3]
    if res is not None:
        pr_w, pr_b = np.asarray(w.pr_w, np.float32), np.asarray(w.pr_b, np.float32)
        pp = pr_b[None, :] + pr_w[None, :, 0] * res[:, None]
        pp = pp + pr_w[None, :, 1] * gate[:, None]
        y = y + pp
    return y.astype(np.float32)


def out_proj(x: np.ndarray, w) -> np.ndarray:
    """out_proj (C -> 1) (sparse_unet.py:258): bias + the quad-order sum of out_w * x (the PMG_EPI_ROUT epilogue)."""
    ow = np.asarray(w.out_w, np.float32).reshape(1, -1)
    return np.float32(np.asarray(w.out_b).reshape(-1)[0]) + quad_sum(ow * x.astype(np.float32))


def linear(x, lin, mode: str, record=None, path=None, acc=np.float64):
    """nn.Linear, out = x @ W^T + b, in the requested arithmetic; `lin` has w (out, in), b, clip. int8: the input
    codes quant_i8(x, 127/clip), then linear_codes; fp16: linear_f16 with sums in `acc`. `record` receives the input
    under `path`."""
    x = np.asarray(x, np.float32)
    if record is not None:
        record[path] = x
    if mode == "fp32":
        return (x @ np.asarray(lin.w, np.float32).T + np.asarray(lin.b, np.float32)).astype(np.float32)
    if mode == "fakequant":
        return (fake_quant(x, lin.clip) @ fake_quant_weight(lin.w).T + np.asarray(lin.b, np.float32)).astype(
            np.float32)
    if mode == "fp16":
        return linear_f16(x, lin, acc=acc)
    return linear_codes(quant_i8(x, act_mult(lin.clip)), lin)


def f16(x):
    """Rounded to fp16 (round to nearest even), as float64."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def linear_f16(x, lin, silu_out: bool = False, acc=np.float64):
    """The teacher's linear: fp16(x) @ fp16(W)^T summed in `acc` (fp64: exactly; fp32: another summation, the spread
    a kernel's own fp32 order may show), rounded to fp32, + b in fp32; with silu_out, SiLU of that, rounded to fp16
    (fuse_proj.0 into fuse_proj.2's input)."""
    y = (f16(x).astype(acc) @ f16(lin.w).astype(acc).T).astype(np.float32) + np.asarray(lin.b, np.float32)
    y = y.astype(np.float32)
    if silu_out:
        from .numerics import silu_f32

        return silu_f32(y).astype(np.float16).astype(np.float32)
    return y


def linear_codes(codes, lin):
    """int8 linear on given input codes: (acc * a) * s_w[n] + b[n], acc the exact int32 product with the int8 weight
    (Refiner.metal:173-250, MODE 0)."""
    q, s = quantize_weight(lin.w)
    acc = np.asarray(codes).astype(np.int64) @ q.astype(np.int64).T
    return dequant(acc, act_scale(lin.clip), s, lin.b)


def linear_silu_codes(x, lin, out_clip):
    """int8 linear, SiLU, and the requantisation of the next layer's input as one epilogue (fuse_proj.0 into
    fuse_proj.2, Refiner.metal:238-242, MODE 1)."""
    q, s = quantize_weight(lin.w)
    codes = quant_i8(np.asarray(x, np.float32), act_mult(lin.clip))
    acc = codes.astype(np.int64) @ q.astype(np.int64).T
    return epilogue_q(acc, act_scale(lin.clip), s, lin.b, act_mult(out_clip))


def resblock(x, nmap, blk, mode: str, trace=None, record=None, path=None, acc=np.float64):
    """SparseResBlock3d.forward (flex_sparse_blocks.py:70-75): h = silu(norm1(x)); conv1; silu; conv2; + x (the
    identity skip: the block keeps its width). `blk` has gamma, beta, w1, b1, w2, b2, clip1, clip2; nmap (M, 27).
    `trace` (a list) receives the block's codes / accumulators (int8) or output; `record` (fp32 / fakequant) the
    inputs of conv1 and conv2 under `path`.conv1 / .conv2."""
    if mode == "int8":
        q_w1, s_w1 = quantize_weight(blk.w1)
        q_w2, s_w2 = quantize_weight(blk.w2)
        x = np.asarray(x, np.float32)
        q1 = rowwise(lambda xb: quant_i8(ln_silu(xb, blk.gamma, blk.beta), act_mult(blk.clip1)), x)
        acc1 = conv_acc_int(q1, nmap, q_w1)
        q2 = rowwise(lambda ab: epilogue_q(ab, act_scale(blk.clip1), s_w1, blk.b1, act_mult(blk.clip2)), acc1)
        acc2 = conv_acc_int(q2, nmap, q_w2)
        out = rowwise(lambda ab, xb: epilogue_r(ab, act_scale(blk.clip2), s_w2, blk.b2, xb), acc2, x)
        if trace is not None:
            trace.append(dict(q1=q1, acc1=acc1, q2=q2, acc2=acc2, x=out))
        return out
    if mode == "fp16":
        from .numerics import silu_f32

        x = np.asarray(x, np.float32)
        h1 = rowwise(lambda xb: ln_silu(xb, blk.gamma, blk.beta).astype(np.float16), x)
        y1 = conv_float(h1.astype(acc), nmap, f16(blk.w1).astype(acc), dtype=acc).astype(np.float32)
        h2 = rowwise(lambda yb: silu_f32(yb + np.asarray(blk.b1, np.float32)).astype(np.float16), y1)
        y2 = conv_float(h2.astype(acc), nmap, f16(blk.w2).astype(acc), dtype=acc).astype(np.float32)
        out = ((y2 + np.asarray(blk.b2, np.float32)) + x).astype(np.float32)
        if trace is not None:
            trace.append(dict(h1=h1, h2=h2, x=out))
        return out
    w1, w2 = np.asarray(blk.w1, np.float32), np.asarray(blk.w2, np.float32)
    h = silu(layer_norm(x, blk.gamma, blk.beta))
    if record is not None:
        record[path + ".conv1"] = h
    if mode == "fakequant":
        h, w1, w2 = fake_quant(h, blk.clip1), fake_quant_weight(blk.w1), fake_quant_weight(blk.w2)
    h = silu(conv_float(h, nmap, w1, blk.b1))
    if record is not None:
        record[path + ".conv2"] = h
    if mode == "fakequant":
        h = fake_quant(h, blk.clip2)
    out = conv_float(h, nmap, w2, blk.b2) + np.asarray(x, np.float32)
    if trace is not None:
        trace.append(dict(x=out))
    return out
