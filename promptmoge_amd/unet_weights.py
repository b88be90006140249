"""Weights of the multi-level sparse U-Net refiner (Sparse3DUNet, moge/model/modules/sparse_unet.py:38-150).

`UNetW` holds one refiner: input_proj / prompt_proj / out_proj (fp32, never quantised: qat.py:118-125), per level
the SparseResBlock3d stages (flex_sparse_blocks.py:50-75), the PoolDown / NearestUp linears
(flex_sparse_blocks.py:78-105), the encoder conditioning encoder_fuse and fuse_proj (sparse_unet.py:81-87), the
bottleneck stage, and the activation clip of every quantised layer's input (qat.py:60-98).

Sources:
  unet_from_state_dict   a Sparse3DUNet state dict, QAT (`.parametrizations.weight.original`, `aq_*.clip`) or plain
                         with the activation clips given
  load_refiner_bin       the Metal engine's export, refiner.bin + refiner.json (promptmoge/export/refiner.py:28-110):
                         int8 weights with their per-output-channel scales are kept exactly as stored (QuantW)
  make_unet_weights      seeded synthetic weights (no checkpoint is available offline)
`save_refiner_bin` writes the same format, so a synthetic refiner round-trips through the loader.
"""
from __future__ import annotations

import dataclasses
import json
from pathlib import Path
from typing import Dict, List, Optional, Sequence, Union

import numpy as np

from .spec import BlockW, quantize_weight as _quantize_master

F32 = np.float32


@dataclasses.dataclass
class QuantW:
    """An int8 weight in the module layout (Co, ...) with its per-output-channel fp32 scale, as refiner.bin stores
    it. Used as an array it is the dequantised q * s."""
    q: np.ndarray
    s: np.ndarray

    @property
    def shape(self):
        return self.q.shape

    def __array__(self, dtype=None, copy=None):
        v = (self.q.astype(F32) * self.s.reshape((-1,) + (1,) * (self.q.ndim - 1))).astype(F32)
        return v if dtype is None else v.astype(dtype)


def quantized(w) -> tuple:
    """(q int8, s fp32 [Co]) of a weight: a QuantW as stored, an fp32 master by the training quantiser
    (WeightFakeQuant, qat.py:52-57)."""
    if isinstance(w, QuantW):
        return np.asarray(w.q, np.int8), np.asarray(w.s, F32)
    return _quantize_master(np.asarray(w, F32))


@dataclasses.dataclass
class LinearW:
    w: Union[np.ndarray, QuantW]  # (out, in)
    b: np.ndarray                 # (out,)
    clip: float = 1.0             # activation clip of the input (quantised layers)


@dataclasses.dataclass
class UNetW:
    channels: List[int]
    factors: List[int]
    enc_channels: int
    in_w: np.ndarray
    in_b: np.ndarray
    pr_w: Optional[np.ndarray]
    pr_b: Optional[np.ndarray]
    out_w: np.ndarray  # (1, C0)
    out_b: np.ndarray  # (1,)
    down: List[List[BlockW]]
    pool: List[LinearW]
    enc: LinearW
    fuse0: LinearW
    fuse2: LinearW
    bott: List[BlockW]
    up: List[LinearW]
    dec: List[List[BlockW]]

    @property
    def levels(self) -> int:
        return len(self.channels)

    @property
    def C(self) -> int:
        return self.channels[0]

    def quantised_layers(self) -> Dict[str, object]:
        """Module path -> layer (BlockW conv pair or LinearW) of every quantised layer, the names enable_refiner_qat
        gives them (qat.py:118-138)."""
        out: Dict[str, object] = {}
        for k, st in enumerate(self.down):
            for j, b in enumerate(st):
                out[f"down_stages.{k}.{j}"] = b
        for k, p in enumerate(self.pool):
            out[f"downsample_blocks.{k}.linear"] = p
        out["encoder_fuse"], out["fuse_proj.0"], out["fuse_proj.2"] = self.enc, self.fuse0, self.fuse2
        for j, b in enumerate(self.bott):
            out[f"bottleneck_stage.{j}"] = b
        for i, u in enumerate(self.up):
            out[f"upsample_blocks.{i}.linear"] = u
        for i, st in enumerate(self.dec):
            for j, b in enumerate(st):
                out[f"up_stages.{i}.{j}"] = b
        return out


# ------------------------------------------------------------------------------------------------ state dict
def unet_from_state_dict(sd, factors: Optional[Sequence[int]] = None,
                         clips: Optional[Dict[str, float]] = None, require_clips: bool = True) -> UNetW:
    """A Sparse3DUNet's weights from its state dict, under the reference's parameter names (sparse_unet.py:81-150,
    flex_sparse_blocks.py:50-105). QAT checkpoints store masters under `.parametrizations.weight.original`
    (torch.nn.utils.parametrize, qat.py:111) and clips in `aq_<module path with '_'>.clip` (qat.py:112-115);
    `clips` ({module path: clip}) overrides them. A quantised layer (qat.py:118-138) with neither raises
    ValueError naming it, so a plain (non-QAT) state dict needs `clips` -- unless `require_clips` is False (the
    fp16 teacher, which quantises nothing: the missing clips are then NaN). `factors` defaults to Sparse3DUNet's
    [2] * (levels - 1)."""
    f32 = lambda t: np.asarray(t.detach().cpu().float().numpy() if hasattr(t, "detach") else t, dtype=F32)

    def has(name):
        base, _, leaf = name.rpartition(".")
        return name in sd or f"{base}.parametrizations.{leaf}.original" in sd

    def get(name):
        if name in sd:
            return f32(sd[name])
        base, _, leaf = name.rpartition(".")
        alt = f"{base}.parametrizations.{leaf}.original"
        if alt in sd:
            return f32(sd[alt])
        raise KeyError(name)

    def clip(path):
        if clips is not None and path in clips:
            return float(clips[path])
        key = "aq_" + path.replace(".", "_") + ".clip"
        if key not in sd:
            if not require_clips:
                return float("nan")
            # the int8 refiner needs every quantised layer's activation clip (export/refiner.py asserts that the
            # observer ran); a default would silently saturate that layer's input
            raise ValueError(f"{path}: quantised layer without an activation clip ({key} is not in the state dict "
                             f"and `clips` does not name it)")
        return float(f32(sd[key]))

    def blocks(prefix):
        out, j = [], 0
        while has(f"{prefix}.{j}.norm1.weight"):
            p = f"{prefix}.{j}"
            if has(f"{p}.skip_connection.weight"):
                raise ValueError(f"{p}: a width-changing SparseResBlock3d is not part of Sparse3DUNet")
            out.append(BlockW(get(f"{p}.norm1.weight"), get(f"{p}.norm1.bias"), get(f"{p}.conv1.weight"),
                              get(f"{p}.conv1.bias"), get(f"{p}.conv2.weight"), get(f"{p}.conv2.bias"),
                              clip(f"{p}.conv1"), clip(f"{p}.conv2")))
            j += 1
        return out

    def lin(path):
        return LinearW(get(f"{path}.weight"), get(f"{path}.bias"), clip(path))

    L = 1
    while has(f"downsample_blocks.{L - 1}.linear.weight"):
        L += 1
    if L < 2:
        raise ValueError("Sparse3DUNet has at least 2 levels (sparse_unet.py:52); no downsample_blocks found")
    in_w = get("input_proj.weight")
    channels = [in_w.shape[0]] + [get(f"downsample_blocks.{k}.linear.weight").shape[0] for k in range(L - 1)]
    enc = lin("encoder_fuse")
    pr = has("prompt_proj.weight")
    return UNetW(
        channels=channels, factors=list(factors) if factors is not None else [2] * (L - 1),
        enc_channels=int(enc.w.shape[1]),
        in_w=in_w, in_b=get("input_proj.bias"),
        pr_w=get("prompt_proj.weight") if pr else None, pr_b=get("prompt_proj.bias") if pr else None,
        out_w=get("out_proj.weight").reshape(1, -1), out_b=get("out_proj.bias").reshape(1),
        down=[blocks(f"down_stages.{k}") for k in range(L)],
        pool=[lin(f"downsample_blocks.{k}.linear") for k in range(L - 1)],
        enc=enc, fuse0=lin("fuse_proj.0"), fuse2=lin("fuse_proj.2"),
        bott=blocks("bottleneck_stage"),
        up=[lin(f"upsample_blocks.{i}.linear") for i in range(L - 1)],
        dec=[blocks(f"up_stages.{i}") for i in range(L - 1)],
    )


# ------------------------------------------------------------------------------------------------ refiner.bin
_DT = {"float16": np.float16, "float32": np.float32, "int8": np.int8}


def load_refiner_bin(directory) -> tuple:
    """refiner.bin + refiner.json as promptmoge/export/refiner.py:28-110 writes them (and Refiner.swift:65-116 reads
    them): named blocks of int8 weights -- convolutions [27][Ci][Co], linears [K][N] -- with fp32 per-output-channel
    scales, fp16 biases and LayerNorm affine, fp32 activation clips, fp16 input/prompt/output projections, and the
    fp32 uv_bias map [C_L][R][C]. One residual block per stage (the export writes stage[0] only, :84-98).
    Returns (UNetW, manifest dict, uv_bias or None); factors are 2 per level (the exported models)."""
    d = Path(directory)
    man = json.loads((d / "refiner.json").read_text())
    raw = (d / "refiner.bin").read_bytes()

    def arr(name):
        e = man["weights"][name]
        dt = np.dtype(_DT[e["dtype"]])
        a = np.frombuffer(raw, dtype=dt, count=int(e["count"]), offset=int(e["offset"]))
        return a.reshape(e["shape"]).copy()

    f = lambda name: arr(name).astype(F32)

    def conv(tag, c):  # [27][Ci][Co] int8 -> module layout (Co, 3, 3, 3, Ci)
        q = arr(f"{tag}.{c}w8")
        co, ci = q.shape[2], q.shape[1]
        qm = np.ascontiguousarray(q.transpose(2, 0, 1)).reshape(co, 3, 3, 3, ci)
        return QuantW(qm, f(f"{tag}.{c}ws").reshape(co))

    def block(tag):
        return BlockW(f(f"{tag}.n1w"), f(f"{tag}.n1b"), conv(tag, "c1"), f(f"{tag}.c1b"), conv(tag, "c2"),
                      f(f"{tag}.c2b"), float(f(f"{tag}.c1clip")[0]), float(f(f"{tag}.c2clip")[0]))

    def qlin(tag):  # [K][N] int8 -> (N, K)
        q = arr(f"{tag}.w8")
        return LinearW(QuantW(np.ascontiguousarray(q.T), f(f"{tag}.ws").reshape(q.shape[1])), f(f"{tag}.b"),
                       float(f(f"{tag}.clip")[0]))

    L = int(man["levels"])
    w = UNetW(
        channels=[int(c) for c in man["channels"]], factors=[2] * (L - 1), enc_channels=int(man["enc_channels"]),
        in_w=np.ascontiguousarray(f("input_proj.w").T), in_b=f("input_proj.b"),
        pr_w=np.ascontiguousarray(f("prompt_proj.w").T) if "prompt_proj.w" in man["weights"] else None,
        pr_b=f("prompt_proj.b") if "prompt_proj.b" in man["weights"] else None,
        out_w=np.ascontiguousarray(f("out_proj.w").T).reshape(1, -1), out_b=f("out_proj.b").reshape(1),
        down=[[block(f"down{k}")] for k in range(L)],
        pool=[qlin(f"pool{k}") for k in range(L - 1)],
        enc=qlin("encoder_fuse"), fuse0=qlin("fuse0"), fuse2=qlin("fuse2"),
        bott=[block("bott")],
        up=[qlin(f"up{i}") for i in range(L - 1)],
        dec=[[block(f"dec{i}")] for i in range(L - 1)],
    )
    uv = f("uv_bias") if "uv_bias" in man["weights"] else None
    return w, man, uv


def save_refiner_bin(w: UNetW, directory, H: int, W: int, depth_resolution: float = 256.0,
                     uv_bias: Optional[np.ndarray] = None) -> None:
    """Writes `w` in the refiner.bin / refiner.json format of promptmoge/export/refiner.py:28-110 (tensor order,
    names, dtypes and layouts of :71-105; one residual block per stage)."""
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    index, chunks, off = {}, [], 0

    def put(name, a, dt):
        nonlocal off
        x = np.ascontiguousarray(np.asarray(a, dtype=F32) if dt != np.int8 else np.asarray(a), dtype=dt)
        index[name] = {"offset": off, "count": int(x.size), "shape": list(x.shape), "dtype": np.dtype(dt).name}
        chunks.append(x.tobytes())
        off += x.nbytes

    def plain(tag, wt, b):
        put(f"{tag}.w", np.asarray(wt, F32).T, np.float16)
        put(f"{tag}.b", b, np.float16)

    def qlin(tag, lin: LinearW):
        q, s = quantized(lin.w)
        put(f"{tag}.w8", q.T, np.int8)
        put(f"{tag}.ws", s, np.float32)
        put(f"{tag}.b", lin.b, np.float16)
        put(f"{tag}.clip", [lin.clip], np.float32)

    def block(tag, b: BlockW):
        put(f"{tag}.n1w", b.gamma, np.float16)
        put(f"{tag}.n1b", b.beta, np.float16)
        for c, wt, bias, cl in (("c1", b.w1, b.b1, b.clip1), ("c2", b.w2, b.b2, b.clip2)):
            q, s = quantized(wt)
            co = q.shape[0]
            put(f"{tag}.{c}w8", q.reshape(co, 27, -1).transpose(1, 2, 0), np.int8)
            put(f"{tag}.{c}ws", s, np.float32)
            put(f"{tag}.{c}b", bias, np.float16)
            put(f"{tag}.{c}clip", [cl], np.float32)

    for st in [*w.down, w.bott, *w.dec]:
        if len(st) != 1:
            raise ValueError("refiner.bin holds one residual block per stage")
    plain("input_proj", w.in_w, w.in_b)
    plain("prompt_proj", w.pr_w if w.pr_w is not None else np.zeros((w.C, 2), F32),
          w.pr_b if w.pr_b is not None else np.zeros(w.C, F32))
    plain("out_proj", w.out_w, w.out_b)
    L = w.levels
    for k in range(L):
        block(f"down{k}", w.down[k][0])
        if k < L - 1:
            qlin(f"pool{k}", w.pool[k])
    qlin("encoder_fuse", w.enc)
    qlin("fuse0", w.fuse0)
    qlin("fuse2", w.fuse2)
    block("bott", w.bott[0])
    for i in range(L - 1):
        qlin(f"up{i}", w.up[i])
        block(f"dec{i}", w.dec[i][0])
    if uv_bias is not None:
        put("uv_bias", uv_bias, np.float32)
    (d / "refiner.bin").write_bytes(b"".join(chunks))
    down = int(np.prod(w.factors))
    man = {"H": H, "W": W, "R": H // down, "C": W // down, "levels": L, "channels": list(w.channels),
           "enc_channels": w.enc_channels, "enc_out": w.channels[-1], "depth_resolution": float(depth_resolution),
           "weights": index}
    (d / "refiner.json").write_text(json.dumps(man, indent=1))


def fp16_exact(w: UNetW) -> UNetW:
    """The refiner as refiner.bin stores it: biases, LayerNorm affine and the three projections rounded to fp16."""
    h = lambda a: None if a is None else np.asarray(a, F32).astype(np.float16).astype(F32)
    blk = lambda b: dataclasses.replace(b, gamma=h(b.gamma), beta=h(b.beta), b1=h(b.b1), b2=h(b.b2))
    lin = lambda l: dataclasses.replace(l, b=h(l.b))
    return dataclasses.replace(
        w, in_w=h(w.in_w), in_b=h(w.in_b), pr_w=h(w.pr_w), pr_b=h(w.pr_b), out_w=h(w.out_w), out_b=h(w.out_b),
        down=[[blk(b) for b in st] for st in w.down], pool=[lin(p) for p in w.pool], enc=lin(w.enc),
        fuse0=lin(w.fuse0), fuse2=lin(w.fuse2), bott=[blk(b) for b in w.bott], up=[lin(u) for u in w.up],
        dec=[[blk(b) for b in st] for st in w.dec])


# ------------------------------------------------------------------------------------------------ synthetic
def make_unet_weights(channels: Sequence[int], enc_channels: int, enc_blocks: Union[int, Sequence[int]] = 1,
                      dec_blocks: Union[int, Sequence[int]] = 1, bottleneck_blocks: int = 1,
                      factors: Optional[Sequence[int]] = None, prompt: bool = True, seed: int = 0) -> UNetW:
    """Seeded synthetic weights of a Sparse3DUNet(in 3, out 1, encoder_channels, channels, ...) (sparse_unet.py:38-
    120): conv weights ~ N(0, 0.05), linear weights ~ N(0, 1/sqrt(fan_in)), biases and LayerNorm shifts ~ N(0,
    0.05), LayerNorm scales ~ 1 + N(0, 0.05); all activation clips 1.0 until calibrated."""
    rng = np.random.default_rng(2000 + seed)
    L = len(channels)
    eb = [enc_blocks] * L if isinstance(enc_blocks, int) else list(enc_blocks)
    db = [dec_blocks] * (L - 1) if isinstance(dec_blocks, int) else list(dec_blocks)
    nrm = lambda *s, sd=0.05: rng.normal(0, sd, size=s).astype(F32)

    def block(C):
        return BlockW(gamma=(1.0 + nrm(C)).astype(F32), beta=nrm(C), w1=nrm(C, 3, 3, 3, C), b1=nrm(C),
                      w2=nrm(C, 3, 3, 3, C), b2=nrm(C))

    def lin(co, ci):
        return LinearW(nrm(co, ci, sd=1.0 / np.sqrt(ci)), nrm(co))

    C0, CL = channels[0], channels[-1]
    return UNetW(
        channels=list(channels), factors=list(factors) if factors is not None else [2] * (L - 1),
        enc_channels=enc_channels,
        in_w=nrm(C0, 3, sd=0.5), in_b=nrm(C0), pr_w=nrm(C0, 2, sd=0.5) if prompt else None,
        pr_b=nrm(C0) if prompt else None, out_w=nrm(1, C0), out_b=nrm(1, sd=0.01),
        down=[[block(channels[k]) for _ in range(eb[k])] for k in range(L)],
        pool=[lin(channels[k + 1], channels[k]) for k in range(L - 1)],
        enc=lin(CL, enc_channels), fuse0=lin(CL, 2 * CL), fuse2=lin(CL, CL),
        bott=[block(CL) for _ in range(bottleneck_blocks)],
        up=[lin(channels[L - 2 - i], channels[L - 1 - i]) for i in range(L - 1)],
        dec=[[block(channels[L - 2 - i]) for _ in range(db[i])] for i in range(L - 1)],
    )
