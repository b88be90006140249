#!/usr/bin/env python3
"""Benchmark of the MI355X refiner step (one JSON line on stdout).

Workload (the headline): a Model-A-shape (480x640) int8 refiner step, K=1: prompt fit
(trimmed LS, 10 trim rounds) -> prompt residual/gate -> voxelise (M = 307,200 voxels) -> column neighbour map ->
input_proj + prompt_proj -> 3 residual blocks = 6 int8 submanifold 3x3x3 conv layers at C=48 -> out_proj -> logz +=
delta, on synthetic seeded inputs (promptmoge_amd.spec) already resident in HBM. One "step" is one replay of the
captured HIP graph of that chain; the metric fit of the refined depth is timed separately (`final_fit_ms`).

    value     active voxels refined per second = M / step time (whole job; one GPU)
    roofline  the dominant kernel of the step (largest time per step): algorithmic bytes per launch / its average
              launch duration. Durations come from HIP events around a captured graph of R back-to-back launches of
              that kernel on the step's own data, recorded on the stream the kernel runs on. `traffic` is the HBM
              bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE passes (see --write-traffic), read from
              profiles/hbm_traffic_modelA.txt when that file is present.
    cpu_baseline  the oracle's restatement of the reference's CPU path (_fallback conv on fake-quantised operands,
              fit_scale_shift with an exact k-th selection) timed on this host: 1 warm-up + median of 5 Model-A steps
    conv_microbench  isolated int8 conv on 1,000,000 surface voxels in 1024^3, C = 64 and 128; beside
              it the same map through the flex_gemm shim's fp16 and bf16 convolutions (fp16_C64 ... bf16_C128;
              the dense bf16 peak equals fp16's)
    measured_peaks   this device's practical HBM copy bandwidth and int8 MFMA rate (pmg_probe_copy / _mfma_i8);
              `roofline.frac` is against the published 8 TB/s, `roofline.frac_measured` against the copy probe
    other_configs    one K-step frame of the fp16 teacher (T) and of the hi-res config (H, with nearest_fill); the
              first U-Net level step of Model A (pool cache, mean pool, nearest upsampling: pool_L0); the prompt
              gauge infer applies after the loop, on Model A's depth and LiDAR (gauge_A)

Other modes (used to produce the committed profiles):
    --kernels-only     launch each per-step kernel --kernel-reps times eagerly (plus a 64 MiB copy for counter
                       calibration) and exit; run under `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE`
    --write-traffic OUT FETCH_DIR WRITE_DIR
                       turn those two counter runs into per-kernel HBM bytes per launch (scaled by the copy kernel's
                       known size) and write them to OUT
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0
# mask-sort window of the microbench's row order per width (0: the whole map). Measured on the 1M-voxel set: C = 64
# (the resident-weight kernel, each wave walks its own taps) runs 0.110 ms at 2^18 rows against 0.123 ms at one
# window (smaller windows keep its gathers in L2); C = 128 (the block walks its chunk's tap union between weight
# staging barriers) runs 0.305 ms at one window against 0.324 ms at 2^18 and 0.37-0.39 ms at 2^14-2^15 (the union
# of a 512-row chunk grows from 11.6 taps at one window to 16.0 at 2^16 and 19.7 at 2^14).
ORDER_WINDOW = {64: 1 << 18, 128: 0}
METRIC = "refiner step latency ms + active voxels/s at 480×640; int8 conv TOPS (% peak)"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_modelA.txt")
CALIB_BYTES = 64 << 20  # the calibration copy: 64 MiB read + 64 MiB written

# kernel-name substrings (as rocprofv3 prints them) for the per-step kernels
KERNEL_SYMBOLS = {
    "fit_prompt": "fit_k",
    "conv_q": "spconv_colv_k<48, 1,",
    "conv_rln": "spconv_colv_k<48, 5,",
    "conv_rout": "spconv_colv_k<48, 6,",
    "input_stage": "input_stage_k<48",
}


def graph_ms(fn, reps, stream):
    """Average duration of fn() in ms: R launches captured into one graph, timed with events on `stream`."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(3):
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / reps)
    return statistics.median(times)


def algorithmic_bytes(cfg):
    """Bytes per launch each per-step kernel must move, from the per-unit figures of the measurement contract:
    conv  M*(Ci + b_out*Co + 108) + 27*Ci*Co  (codes in, outputs, a 27-entry int32 map per voxel, weights; the
          column conv derives the map from 4-byte keys instead of reading 108 B, see `minimal` below)
    fit   18 B per element per trim round (z, target, mask for the sums; again for the residual pass) + 9 B final.
    `minimal` lists what these kernels actually have to read and write once."""
    M, C, it = cfg.M, cfg.C, cfg.fit_iters
    wb = 27 * C * C
    contract = {
        "fit_prompt": M * (18 * it + 9),
        "conv_q": M * (C + C + 108) + wb,
        "conv_rln": M * (C + 4 * C + 4 * C + C + 108) + wb,  # + fp32 residual in/out, next codes
        "conv_rout": M * (C + 4 * C + 12 + 12 + 108) + wb,  # + fp32 residual in, point map in/out
    }
    minimal = {
        "fit_prompt": M * 12,
        "conv_q": M * (C + 4 + C) + wb,
        "conv_rln": M * (C + 4 + 4 * C + 4 * C + C) + wb,
        "conv_rout": M * (C + 4 + 4 * C + 12 + 12) + wb,
    }
    return contract, minimal


def read_traffic():
    """Per-kernel HBM bytes per launch from profiles/hbm_traffic_modelA.txt (lines `traffic <name> <fetch> <write>`)."""
    out = {}
    if not os.path.exists(TRAFFIC_FILE):
        return out
    for line in open(TRAFFIC_FILE):
        p = line.split()
        if len(p) == 4 and p[0] == "traffic":
            out[p[1]] = (float(p[2]), float(p[3]))
    return out


def write_traffic(out_path, fetch_dir, write_dir):
    """Averages FETCH_SIZE / WRITE_SIZE (KiB per dispatch) per kernel over two rocprofv3 --pmc runs of
    `bench.py --kernels-only`, scales each counter so that the calibration copy reads and writes CALIB_BYTES,
    and writes the per-kernel HBM bytes per launch."""

    def load(d, counter):
        vals = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] == counter:
                    vals.setdefault((r["Kernel_Name"], r["Grid_Size"]), []).append(float(r["Counter_Value"]) * 1024)
        return vals

    fv, wv = load(fetch_dir, "FETCH_SIZE"), load(write_dir, "WRITE_SIZE")

    def calib(vals):
        # the copy kernel is the only dispatch moving about CALIB_BYTES; take the largest per-dispatch value
        # among kernels whose name marks them as copies
        cands = [statistics.median(v) for (k, _), v in vals.items() if "copy" in k.lower() or "elementwise" in k]
        return CALIB_BYTES / max(cands)

    fs, ws = calib(fv), calib(wv)
    lines = [f"# HBM traffic per launch, Model A (480x640, C=48), from rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE",
             f"# scale factors from a {CALIB_BYTES} B copy: FETCH_SIZE x{fs:.4f}, WRITE_SIZE x{ws:.4f}",
             "# commands (GPU box, from /tmp with TMPDIR=/tmp), then this summary:",
             "#   rocprofv3 --pmc FETCH_SIZE --output-format csv -d <F> -o k -- python3 <repo>/bench.py --kernels-only",
             "#   rocprofv3 --pmc WRITE_SIZE --output-format csv -d <W> -o k -- python3 <repo>/bench.py --kernels-only",
             "#   python3 <repo>/bench.py --write-traffic <this file> <F> <W>",
             "# columns: traffic <kernel> <fetch bytes> <write bytes>"]
    for name, sym in KERNEL_SYMBOLS.items():
        f = [statistics.median(v) for (k, _), v in fv.items() if sym in k]
        w = [statistics.median(v) for (k, _), v in wv.items() if sym in k]
        if f and w:
            lines.append(f"traffic {name} {f[0] * fs:.0f} {w[0] * ws:.0f}")
    with open(out_path, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def setup(cfg_name):
    import torch

    from promptmoge_amd import ops, spec
    from promptmoge_amd.refiner import RefinerStep

    dev = torch.device("cuda:0")
    cfg = spec.CONFIGS[cfg_name]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    stream = torch.cuda.Stream()
    env = {"cfg": cfg, "sc": sc, "w": w, "stream": stream}
    with torch.cuda.stream(stream):
        P = torch.from_numpy(sc.points[None].copy()).to(dev)
        env.update(P=P, Pout=torch.empty_like(P), L=torch.from_numpy(sc.lidar[None].copy()).to(dev),
                   Cf=torch.from_numpy(sc.conf[None].copy()).to(dev))
        step = RefinerStep(w, 1, cfg.H, cfg.W, precision=cfg.precision, fit_iters=cfg.fit_iters)
        step(env["P"], env["L"], env["Cf"], out=env["Pout"])
        step.check()
        if cfg.precision != "int8":  # the single-kernel timings below are int8 (config A); fits only
            torch.cuda.synchronize()
            env["step"] = step
            return env
        zq, _, _ = ops.voxelize(P[..., 2:], 256.0, stride=3, shape=(1, cfg.H, cfg.W))
        x = step.buffer("x").clone()
        b0, b1 = step.weights.blocks[0], step.weights.blocks[-1]
        q1 = ops.ln_silu_quant(x, b0["gamma"], b0["beta"], b0["m1"])
        q2 = ops.spconv_col(q1, zq, b0["w1"], ops.EPI_Q, a_scale=b0["a1"], w_scale=b0["s1"], bias=b0["b1"],
                            out_mult=b0["m2"])
        xr, nq, Pk = x.clone(), torch.empty_like(q1), torch.empty_like(P)
        torch.cuda.synchronize()
    env["step"] = step
    env["kernels"] = {
        "fit_prompt": lambda: ops.fit_prompt(P, env["L"], env["Cf"], iters=cfg.fit_iters),
        "conv_q": lambda: ops.spconv_col(q1, zq, b0["w1"], ops.EPI_Q, a_scale=b0["a1"], w_scale=b0["s1"],
                                         bias=b0["b1"], out_mult=b0["m2"], out=q2),
        "conv_rln": lambda: ops.spconv_col(q2, zq, b0["w2"], ops.EPI_RLN, a_scale=b0["a2"], w_scale=b0["s2"],
                                           bias=b0["b2"], skip=xr, out=xr, ln_gamma=b1["gamma"], ln_beta=b1["beta"],
                                           next_mult=b1["m1"], next_q=nq),
        "conv_rout": lambda: ops.spconv_col(q2, zq, b1["w2"], ops.EPI_ROUT, a_scale=b1["a2"], w_scale=b1["s2"],
                                            bias=b1["b2"], skip=x, out_w=step.weights.out_w,
                                            out_b=step.weights.out_b, points=P, points_out=Pk),
    }
    return env


def kernels_only(args):
    import torch

    env = setup(args.config)
    with torch.cuda.stream(env["stream"]):
        for _ in range(3):
            env["step"](env["P"], env["L"], env["Cf"], out=env["Pout"])
        for name, fn in env["kernels"].items():
            for _ in range(args.kernel_reps):
                fn()
        a = torch.empty(CALIB_BYTES // 4, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        a.fill_(1.0)
        for _ in range(args.kernel_reps):
            b.copy_(a)
        torch.cuda.synchronize()
    print("kernels-only done", flush=True)
    return 0


def measured_peaks(stream):
    """The device's practical peaks with the kernels' instruction forms (pmg_probe_copy: 16-byte vector copy of
    1 GiB, read + write bytes; pmg_probe_mfma_i8: register-only v_mfma_i32_16x16x64_i8 loops at 8 and 16 waves
    per CU, the better of the two). Median of 3 event-timed runs each."""
    import ctypes as C

    import torch

    from promptmoge_amd._lib import call

    nbytes = 1 << 30
    with torch.cuda.stream(stream):
        a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        a.fill_(1)
        sink = torch.zeros(1, dtype=torch.int32, device="cuda")
        sp = C.c_void_p(stream.cuda_stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

        def timed(fn):
            fn()
            ts = []
            for _ in range(3):
                e0.record(stream)
                fn()
                e1.record(stream)
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1))
            return statistics.median(ts)

        t = timed(lambda: call("pmg_probe_copy", a.data_ptr(), b.data_ptr(), nbytes, sp))
        hbm = 2 * nbytes / (t * 1e-3) / 1e9
        best = 0.0
        iters = 2048
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        for wpc in (8, 16):
            t = timed(lambda: call("pmg_probe_mfma_i8", iters, wpc, sink.data_ptr(), sp))
            ops = cus * wpc * iters * 16 * 32768.0
            best = max(best, ops / (t * 1e-3) / 1e12)
        del a, b
    return {"hbm_copy_gbs": round(hbm, 1), "int8_mfma_tops": round(best, 1)}

def microbench(stream):
    import torch

    from promptmoge_amd import ops, spec

    dev = torch.device("cuda:0")
    coords = spec.make_voxels(1_000_000, 1024, seed=21)
    with torch.cuda.stream(stream):
        cd = torch.from_numpy(coords).to(dev)
        shape = (1, 1024, 1024, 1024)
        ntu, tmu, nru, rmu = ops.nmap_hash(cd, shape, rows=True, row_mask=True)
        torch.cuda.synchronize()
        hash_ms = graph_ms(lambda: ops.nmap_hash(cd, shape, row_mask=True), 5, stream)
        # the same map from the (b, x, y) columns' row runs: the set is in _linearise order (as voxelisation and
        # pool caches leave it); the order is checked on the device inside the timed call, and its status read after
        sws = ops.sorted_workspace(shape, dev)
        nts = ops.nmap_sorted(cd, shape, row_mask=True, workspace=sws)[0]
        torch.cuda.synchronize()
        sorted_ms = graph_ms(lambda: ops.nmap_sorted(cd, shape, row_mask=True, workspace=sws), 5, stream)
        if ops.sorted_status(sws) != 0 or not torch.equal(nts, ntu):
            raise RuntimeError("microbench: the sorted map differs from the hash map")
        pu = int((ntu >= 0).sum().item())
        M = coords.shape[0]
        micro = {"voxels": int(M), "pairs": pu, "mean_active_taps": round(pu / M, 3), "hash_map_ms": round(hash_ms, 4),
                 "hash_map_gbs": round((16 * M + 108 * M) / (hash_ms * 1e-3) / 1e9, 1),
                 "sorted_map_ms": round(sorted_ms, 4),
                 "sorted_map_gbs": round((16 * M + 108 * M) / (sorted_ms * 1e-3) / 1e9, 1)}
        g = torch.Generator(device="cpu").manual_seed(5)
        for Cm in (64, 128):
            # the map's processing order for this width (rows sorted by tap mask within windows of ORDER_WINDOW[Cm]
            # rows, the map permuted into it): built once per map, like the map itself, and read by every
            # convolution of that width on it; its build time is reported beside the convolution's
            win = ORDER_WINDOW[Cm]
            order, otm, nmo = ops.row_order(rmu, nru, window=win)
            torch.cuda.synchronize()
            order_ms = graph_ms(lambda: ops.row_order(rmu, nru, window=win), 5, stream)
            xm = torch.randint(-127, 128, (M, Cm), generator=g, dtype=torch.int8).to(dev)
            wm = torch.randint(-127, 128, (Cm, 3, 3, 3, Cm), generator=g, dtype=torch.int8).to(dev)
            sm = torch.full((Cm,), 1e-4, device=dev)
            om = torch.empty((M, Cm), dtype=torch.int8, device=dev)
            # the microbenchmark's epilogue: per-channel requantisation q = clamp(rint(acc * m[n]), +-127); rows in
            # the map's processing order (the caller's order timed beside it)
            t = graph_ms(lambda: ops.spconv_i8_ordered(xm, nmo, order, otm, wm, ops.EPI_QLIN, w_scale=sm, out=om),
                         5, stream)
            t_u = graph_ms(lambda: ops.spconv_i8(xm, ntu, tmu, wm, ops.EPI_QLIN, w_scale=sm, out=om), 5, stream)
            tops = 2 * Cm * Cm * pu / (t * 1e-3) / 1e12
            gain = t_u - t
            micro[f"C{Cm}"] = {"ms": round(t, 4), "tops": round(tops, 2), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                               "ms_caller_order": round(t_u, 4), "order_window": win or M,
                               "row_order_ms": round(order_ms, 4),
                               # one convolution on a fresh map, its order built first
                               "ms_with_order_build": round(t + order_ms, 4),
                               # convolutions of this width on one map that repay the order's build
                               "order_break_even_convs": round(order_ms / gain, 1) if gain > 0 else None}
            del order, otm, nmo
        # the same map through the flex_gemm shim's fp16 and bf16 paths (SubmanifoldConv3d on fp16 / bf16
        # features: fp16 / bf16 MFMA, fp32 accumulators, caller's row order)
        for name, dt, conv in (("fp16", torch.float16, ops.spconv_f16), ("bf16", torch.bfloat16, ops.spconv_bf16)):
            for Cm in (64, 128):
                xh = (torch.randn(M, Cm, generator=g) * 0.5).to(dt).to(dev)
                wh = (torch.randn(Cm, 3, 3, 3, Cm, generator=g) * 0.05).to(dt).to(dev)
                oh = torch.empty((M, Cm), dtype=torch.float32, device=dev)
                t = graph_ms(lambda: conv(xh, ntu, tmu, wh, ops.EPI_ACC, out=oh), 5, stream)
                tf = 2 * Cm * Cm * pu / (t * 1e-3) / 1e12
                micro[f"{name}_C{Cm}"] = {"ms": round(t, 4), "tflops": round(tf, 2),
                                          "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4)}
    return micro


def fit_trace(args):
    """The metric fit's own per-round record: block 0 of fit_k writes, into the workspace header, the wall clock
    (100 MHz) at the launch, after the first solve and after every trim round, with the round's selection path
    (bracket, window pass, radix passes, and the fallbacks between them), its histogram passes, its candidate count
    and threshold, and the number of rounds run (the loop stops at a fixed point). Prints one line per round for the prompt fit and the final fit of
    the configuration, on its input point map and on the map one refiner step made (the last of 20 runs each). A
    library built with PMG_FIT_PHASE_TRACE=1 (python -m promptmoge_amd.build) also records the phases of each
    round, which are printed after it."""
    import numpy as np
    import torch

    from promptmoge_amd import ops

    env = setup(args.config)
    cfg = env["cfg"]
    P, L, Cf, Pr = env["P"], env["L"], env["Cf"], env["Pout"]
    names = {0: "bracket", 1: "bracket missed -> radix", 2: "radix", 4: "window", 5: "bracket missed -> window",
             6: "window missed -> radix", 7: "bracket, window missed -> radix"}
    with torch.cuda.stream(env["stream"]):
        # on the input point map, and on the map one refiner step made (what the final fit and the prompt fits of
        # later steps see)
        for name, run in (("prompt fit", lambda: ops.fit_prompt(P, L, Cf, iters=cfg.fit_iters)),
                          ("final fit", lambda: ops.fit_final(P, L, Cf, iters=cfg.fit_iters)),
                          ("prompt fit on the refined map", lambda: ops.fit_prompt(Pr, L, Cf, iters=cfg.fit_iters)),
                          ("final fit on the refined map", lambda: ops.fit_final(Pr, L, Cf, iters=cfg.fit_iters))):
            for _ in range(20):
                run()
            torch.cuda.synchronize()
            ws = next(iter(ops._FIT_WS.values()))
            tr = ws[128:128 + 4096].cpu().numpy().view(np.uint32)
            t0, t1 = int(tr[129]), int(tr[128])
            print(f"# {name}, config {cfg.name} ({cfg.H}x{cfg.W}, iters {cfg.fit_iters}); times in us from the launch")
            print(f"load + first solve {((t1 - t0) & 0xffffffff) / 100.0:8.2f}")
            prev = t1
            for it in range(int(tr[130])):
                t = int(tr[2 * it + 1])
                dt = ((t - prev) & 0xffffffff) / 100.0
                thr = int(tr[768 + it])
                move = f"{thr - int(tr[768 + it - 1]):+10d}" if it else " " * 10
                code = int(tr[2 * it])
                pname = names.get(code & 7, "?") + (" + one-value threshold" if code & 8 else "")
                line = (f"round {it:2d} {dt:8.2f}  path {pname:32s} passes {(code >> 4) & 15}  "
                        f"candidates {code >> 8:5d}  threshold {np.uint32(thr).view(np.float32):.6e} "
                        f"(move {move} ulps)")
                mk = [int(v) for v in tr[256 + it * 8: 256 + it * 8 + 7]]
                if it < 32 and any(mk):  # phase marks: a library built with PMG_FIT_PHASE_TRACE=1
                    d = [((mk[k + 1] - mk[k]) & 0xffffffff) / 100.0 for k in range(6)]
                    line += (f"  | before stage {((mk[0] - prev) & 0xffffffff) / 100.0:.2f} publish {d[0]:.2f} "
                             f"barrier {d[1]:.2f} totals {d[2]:.2f} candload {d[3]:.2f} select {d[4]:.2f} "
                             f"solve {d[5]:.2f}")
                print(line)
                prev = t
            print(f"total (block 0) {((prev - t0) & 0xffffffff) / 100.0:8.2f}", flush=True)
    return 0


def unet_bench(stream, reps=20, channels=(32, 64, 128, 256, 256), precision="int8"):
    """The multi-level refiner (UNetRefiner, pmg_unet_*) at Model A's size: a 5-level Sparse3DUNet with the deployed
    int8 channels [32, 64, 128, 256, 256] (or the fp16 teacher's stock [32, 64, 128, 256, 512]), one block per
    stage, encoder 1024 channels on the 30 x 40 token grid, prompt features and encoder bias map; one forward =
    level structure + maps + all layers (one captured graph)."""
    import numpy as np
    import torch

    from promptmoge_amd import spec
    from promptmoge_amd import unet_weights as uw
    from promptmoge_amd.unet import UNetRefiner

    cfg = spec.CONFIGS["A"]
    sc = spec.make_scene(cfg)
    H, W = cfg.H, cfg.W
    w = uw.make_unet_weights(list(channels), 1024, seed=1)
    for layer in w.quantised_layers().values():  # clips of the right scale for these weights (timing only)
        if hasattr(layer, "clip1"):
            layer.clip1, layer.clip2 = 3.0, 2.0
        else:
            layer.clip = 3.0
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0)
    M = H * W
    with torch.cuda.stream(stream):
        feats = torch.from_numpy(sc.points.reshape(M, 3).copy()).to(dev)
        enc = torch.from_numpy(rng.normal(0, 1, (1, 1024, H // 16, W // 16)).astype(np.float32)).to(dev)
        bias = torch.from_numpy(rng.normal(0, 0.1, (1, channels[-1], H // 16, W // 16)).astype(np.float32)).to(dev)
        pf = torch.from_numpy(np.stack([rng.normal(0, 0.05, M), rng.uniform(0, 1, M)], 1).astype(np.float32)).to(dev)
        mod = UNetRefiner(w, precision=precision)
        shape = torch.Size([1, H, W, 1024, 3])
        for _ in range(3):
            mod(feats, None, shape, enc, prompt_feats=pf, encoder_bias_map=bias)
        torch.cuda.synchronize()
        counts = [int(c) for c in mod.buffer("counts", 0).cpu()]
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            mod(feats, None, shape, enc, prompt_feats=pf, encoder_bias_map=bias)
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    return {"workload": f"A-shape 5-level {precision} Sparse3DUNet {list(channels)}, 1 block per stage, encoder "
                        f"1024 x 30x40 tokens, prompt + bias map; forward incl. level structure (keys from depth)",
            "voxels_per_level": counts, "ms": round(ms, 4), "voxels_per_s": round(M / (ms * 1e-3), 1)}


def unet_step_bench(stream, reps=20):
    """One fused refine step with the multi-level int8 refiner (UNetStep, pmg_unet_step) at Model A's size: prompt
    fit (10 rounds) -> residual/gate -> voxelise -> the 5-level U-Net of unet_bench -> logz + delta -> final metric
    fit (10 rounds) -> post_depth, one captured graph on the stream (the inputs resident, in place)."""
    import numpy as np
    import torch

    from promptmoge_amd import spec
    from promptmoge_amd import unet_weights as uw
    from promptmoge_amd.unet import UNetStep

    cfg = spec.CONFIGS["A"]
    sc = spec.make_scene(cfg)
    H, W = cfg.H, cfg.W
    w = uw.make_unet_weights([32, 64, 128, 256, 256], 1024, seed=1)
    for layer in w.quantised_layers().values():  # clips of the right scale for these weights (timing only)
        if hasattr(layer, "clip1"):
            layer.clip1, layer.clip2 = 3.0, 2.0
        else:
            layer.clip = 3.0
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0)
    res = {"workload": "A-shape 5-level int8 refine step: prompt fit + residual/gate + voxelise + Sparse3DUNet "
                       "[32, 64, 128, 256, 256] (1 block per stage, encoder 1024 x 30x40, bias map) + logz update "
                       "+ final metric fit + post_depth, fit iters 10, one captured graph"}
    with torch.cuda.stream(stream):
        P0 = torch.from_numpy(sc.points[None].copy()).to(dev)
        L = torch.from_numpy(sc.lidar[None].copy()).to(dev)
        Cf = torch.from_numpy(sc.conf[None].copy()).to(dev)
        enc = torch.from_numpy(rng.normal(0, 1, (1, 1024, H // 16, W // 16)).astype(np.float32)).to(dev)
        bias = torch.from_numpy(rng.normal(0, 0.1, (1, 256, H // 16, W // 16)).astype(np.float32)).to(dev)
        out = torch.empty_like(P0)
        for key, final in (("ms", True), ("ms_without_final_fit", False)):
            step = UNetStep(w, 1, H, W, fit_iters=cfg.fit_iters, final_fit=final, post_depth=final, device=dev)
            for _ in range(3):
                step(P0, L, Cf, enc, bias, out=out)
            step.check()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                step(P0, L, Cf, enc, bias, out=out)
            e1.record(stream)
            torch.cuda.synchronize()
            step.check()
            res[key] = round(e0.elapsed_time(e1) / reps, 4)
            step.close()
    res["voxels_per_s"] = round(H * W / (res["ms"] * 1e-3), 1)
    return res


def frame_bench(name, stream, reps=10):
    """One frame of a K-step configuration: K refine steps (each with its prompt fit, voxel keys and stencil
    rebuilt, v3.py:537-578) and the final metric fit after the last one. H also times the GPU nearest_fill of its
    LiDAR prompt with 20 % holes (model.py:61-72)."""
    import numpy as np
    import torch

    from promptmoge_amd import ops, spec
    from promptmoge_amd.refiner import RefinerStep

    dev = torch.device("cuda:0")
    cfg = spec.CONFIGS[name]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    K = cfg.steps
    out = {"workload": f"{cfg.name}: {cfg.H}x{cfg.W} {cfg.precision} refiner, K={K} steps + final fit, C={cfg.C}, "
                       f"{2 * cfg.n_blocks} conv layers, fit iters {cfg.fit_iters}", "voxels_per_step": cfg.M}
    with torch.cuda.stream(stream):
        P0 = torch.from_numpy(sc.points[None].copy()).to(dev)
        bufs = [torch.empty_like(P0), torch.empty_like(P0)]
        L = torch.from_numpy(sc.lidar[None].copy()).to(dev)
        Cf = torch.from_numpy(sc.conf[None].copy()).to(dev)
        mid = RefinerStep(w, 1, cfg.H, cfg.W, precision=cfg.precision, fit_iters=cfg.fit_iters)
        last = RefinerStep(w, 1, cfg.H, cfg.W, precision=cfg.precision, fit_iters=cfg.fit_iters, final_fit=True)

        def frame():
            src = P0
            for k in range(K):
                dst = bufs[k % 2]
                (last if k == K - 1 else mid)(src, L, Cf, out=dst)
                src = dst

        for _ in range(3):
            frame()
        mid.check()
        last.check()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            frame()
        e1.record(stream)
        torch.cuda.synchronize()
        fms = e0.elapsed_time(e1) / reps
        mid.check()
        last.check()
        out.update(ms_per_frame=round(fms, 4), ms_per_step=round(fms / K, 4),
                   voxels_per_s=round(K * cfg.M / (fms * 1e-3), 1))
        if cfg.holes > 0:
            rng = np.random.default_rng(cfg.seed + 7)
            raw = np.where(rng.random(sc.lidar.shape) < cfg.holes, 0.0, sc.lidar).astype(np.float32)
            Lr = torch.from_numpy(raw[None]).to(dev)
            Cr = Cf.clone()
            out["nearest_fill_ms"] = round(graph_ms(lambda: ops.nearest_fill(Lr, Cr), 20, stream), 4)
    return out


def pool_bench(stream, reps=20):
    """The first U-Net level step of Model A (flex_sparse_blocks.py:78-105): the 307,200 level-0 voxels pooled by 2
    (pool cache: sort, unique, parent, segments -- with the host read of the output count the reference also
    makes), the C=48 mean pooling, and the nearest upsampling back."""
    import numpy as np
    import torch

    from promptmoge_amd import ops, spec

    dev = torch.device("cuda:0")
    cfg = spec.CONFIGS["A"]
    sc = spec.make_scene(cfg)
    with torch.cuda.stream(stream):
        # level-0 voxels (v3.py:305-344) from the GPU voxeliser: (0, i, j, zq - zmin) in raster order
        P = torch.from_numpy(sc.points[None].copy()).to(dev)
        zq, zmin, zmax = ops.voxelize(P[..., 2:], 256.0, stride=3, shape=(1, cfg.H, cfg.W))
        Z = int(zmax[0] - zmin[0]) + 1
        ii, jj = torch.meshgrid(torch.arange(cfg.H, device=dev), torch.arange(cfg.W, device=dev), indexing="ij")
        ct = torch.stack([torch.zeros_like(ii), ii, jj, (zq[0] - zmin[0]).long()], -1).reshape(-1, 4)
        ct = ct.to(torch.int32).contiguous()
        shape = (1, cfg.H, cfg.W, Z)
        osh = [1, (cfg.H + 1) // 2, (cfg.W + 1) // 2, (Z + 1) // 2]
        f = torch.from_numpy(np.random.default_rng(1).normal(size=(cfg.M, cfg.C)).astype(np.float32)).to(dev)
        oc, parent, seg, offs = ops.pool_cache(ct, shape, (2, 2, 2), osh)
        n = oc.shape[0]
        times = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ops.pool_cache(ct, shape, (2, 2, 2), osh)
            times.append((time.perf_counter() - t0) * 1e3)
        pooled = ops.sparse_pool(f, seg, offs, n)
        pool_ms = graph_ms(lambda: ops.sparse_pool(f, seg, offs, n), 20, stream)
        up_ms = graph_ms(lambda: ops.sparse_upsample(pooled, parent), 20, stream)
    return {"workload": f"A level 0 -> 1: {cfg.M} voxels pooled by 2 -> {n}, C={cfg.C} fp32 mean pool, nearest up",
            "voxels_in": cfg.M, "voxels_out": int(n), "cache_ms": round(statistics.median(times), 4),
            "pool_ms": round(pool_ms, 4), "upsample_ms": round(up_ms, 4),
            "pool_gbs": round((cfg.M * cfg.C * 4 + n * cfg.C * 4 + cfg.M * 4 + n * 8) / (pool_ms * 1e-3) / 1e9, 1),
            "upsample_gbs": round((cfg.M * cfg.C * 4 * 2 + cfg.M * 4) / (up_ms * 1e-3) / 1e9, 1)}


def gauge_bench(stream):
    """The prompt gauge infer applies after the refine loop (gauge_poly=2, v3.py:841-853) on Model A's refined
    depth with its 480x640 LiDAR prompt: pooled inputs, 3 IRLS rounds on one CU, the full-resolution correction."""
    import numpy as np
    import torch

    from promptmoge_amd import ops, spec

    dev = torch.device("cuda:0")
    cfg = spec.CONFIGS["A"]
    sc = spec.make_scene(cfg)
    with torch.cuda.stream(stream):
        depth = torch.from_numpy(np.exp(sc.points[..., 2].astype(np.float64)).astype(np.float32)[None]).to(dev)
        lidar = torch.from_numpy(sc.lidar[None].copy()).to(dev)
        conf = torch.from_numpy(sc.conf[None].copy()).to(dev)
        ms = graph_ms(lambda: ops.gauge_poly(depth, lidar, conf, 2, 3), 10, stream)
    return {"workload": f"A: prompt gauge, degree 2, 3 IRLS rounds, depth {cfg.H}x{cfg.W}, LiDAR {cfg.H}x{cfg.W}",
            "ms": round(ms, 4)}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_time(cfg, sc, w, reps=5):
    """Median seconds of `reps` CPU steps (after one warm-up) of the torch restatement of the _fallback path."""
    from oracle import torch_port

    run = lambda: torch_port.step(sc.points[None], sc.lidar[None], sc.conf[None], w, iters=cfg.fit_iters)
    run()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(env):
    """The reference's CPU path (the _fallback flex_gemm ops, QAT fake quantisation, kthvalue fit) restated op for op
    in torch (oracle/torch_port.py), on all the host's cores: 1 warm-up, median of 5 steps of the workload (the
    top-level figures), and the same for config B (the reference's own CPU case)."""
    import torch

    from promptmoge_amd import spec

    cfg, sc, w = env["cfg"], env["sc"], env["w"]
    nproc = os.cpu_count() or 1
    prev = torch.get_num_threads()
    torch.set_num_threads(nproc)
    try:
        tc = _cpu_time(cfg, sc, w)
        cfg_b = spec.CONFIGS["B"]
        sc_b = spec.make_scene(cfg_b)
        tb = _cpu_time(cfg_b, sc_b, spec.refiner_for(cfg_b, sc_b))
        threads = torch.get_num_threads()
    finally:
        torch.set_num_threads(prev)
    what = ("the reference's _fallback path restated op for op in torch on the CPU (per-tap index_select / mm / "
            f"index_add_, QAT fake quantisation, kthvalue fit), torch.set_num_threads({nproc})")
    return {"value": round(cfg.M / tc, 1), "unit": "voxels/s", "cores": int(threads), "kind": "port",
            "nproc": nproc, "threads": int(threads), "cpu_model": _cpu_model(),
            "sample": f"1 warm-up + median of 5 steps of config {cfg.name} ({cfg.M} voxels each): {what}",
            "ms_per_step": round(tc * 1e3, 1),
            "configs": {"B": {"workload": f"B: {cfg_b.H}x{cfg_b.W} int8 refiner step K=1, C={cfg_b.C}, "
                                          f"{2 * cfg_b.n_blocks} conv layers, fit iters {cfg_b.fit_iters}",
                              "value": round(cfg_b.M / tb, 1), "unit": "voxels/s", "ms_per_step": round(tb * 1e3, 1),
                              "sample": f"1 warm-up + median of 5 steps ({cfg_b.M} voxels each)"}}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="A", choices=["A", "B", "H", "T"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-micro", action="store_true", help="skip the 1M-voxel conv microbench")
    ap.add_argument("--no-others", action="store_true", help="skip the K-step T and H frame timings")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--kernels-only", action="store_true")
    ap.add_argument("--fit-trace", action="store_true",
                    help="print the metric fit's per-round phase trace (prompt and final fit of config A)")
    ap.add_argument("--micro-only", action="store_true",
                    help="run only the 1M-voxel map and conv microbench (for counter collection) and print it")
    ap.add_argument("--write-traffic", nargs=3, metavar=("OUT", "FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--other", choices=["T", "H", "unet_A", "unet_A_step", "unet_T"],
                    help="time only this other configuration (K-step frame, or the multi-level U-Net) and print it")
    args = ap.parse_args()
    if args.write_traffic:
        write_traffic(*args.write_traffic)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the refiner step is per frame and this build uses no collectives); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch

    sys.path.insert(0, ROOT)
    if args.kernels_only:
        return kernels_only(args)
    if args.config == "T" and not args.fit_trace:
        ap.error("--config T serves --fit-trace only; the T frame is timed by --other T")
    if args.fit_trace:
        return fit_trace(args)
    if args.micro_only:
        print(json.dumps({"conv_microbench": microbench(torch.cuda.Stream())}), flush=True)
        return 0
    if args.other:
        s = torch.cuda.Stream()
        res = {"unet_A": unet_bench, "unet_A_step": unet_step_bench,
               "unet_T": lambda st: unet_bench(st, channels=(32, 64, 128, 256, 512), precision="fp16")}.get(
            args.other, lambda st: frame_bench(args.other, st))(s)
        print(json.dumps({args.other: res}), flush=True)
        return 0
    from promptmoge_amd.refiner import RefinerStep

    env = setup(args.config)
    cfg, stream, step = env["cfg"], env["stream"], env["step"]
    P, Pout, L, Cf = env["P"], env["Pout"], env["L"], env["Cf"]
    M, C = cfg.M, cfg.C
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            step(P, L, Cf, out=Pout)
        step.check()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            step(P, L, Cf, out=Pout)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_time(e1) / args.steps
        step.check()

        stepf = RefinerStep(env["w"], 1, cfg.H, cfg.W, precision=cfg.precision, fit_iters=cfg.fit_iters,
                            final_fit=True)
        for _ in range(5):
            stepf(P, L, Cf, out=Pout)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(50):
            stepf(P, L, Cf, out=Pout)
        e1.record(stream)
        torch.cuda.synchronize()
        ms_with_final = e0.elapsed_time(e1) / 50
        stepf.check()

        kern = {k: graph_ms(fn, args.kernel_reps, stream) for k, fn in env["kernels"].items()}
    nb = cfg.n_blocks
    per_step = {"fit_prompt": kern["fit_prompt"], "conv_q": nb * kern["conv_q"],
                "conv_rln": (nb - 1) * kern["conv_rln"], "conv_rout": kern["conv_rout"]}
    per_step["input_stage_and_gaps"] = max(ms - sum(per_step.values()), 0.0)
    dominant = max(kern, key=lambda k: per_step[k])
    contract, minimal = algorithmic_bytes(cfg)
    ach = contract[dominant] / (kern[dominant] * 1e-3) / 1e9
    traffic = read_traffic().get(dominant)
    roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None if traffic is None else int(sum(traffic)),
                "kernel": dominant, "algorithmic_bytes": int(contract[dominant]),
                "minimal_bytes": int(minimal[dominant]), "avg_launch_ms": round(kern[dominant], 5)}

    peaks = measured_peaks(stream)
    roofline["measured_peak"] = peaks["hbm_copy_gbs"]
    roofline["frac_measured"] = round(ach / peaks["hbm_copy_gbs"], 4)
    micro = None if args.no_micro else microbench(stream)
    if micro:
        for Cm in ("C64", "C128"):
            micro[Cm]["frac_measured_int8"] = round(micro[Cm]["tops"] / peaks["int8_mfma_tops"], 4)
    others = None if args.no_others else {n: frame_bench(n, stream) for n in ("T", "H")}
    if others is not None:
        others["pool_L0"] = pool_bench(stream)
        others["gauge_A"] = gauge_bench(stream)
        others["unet_A"] = unet_bench(stream)
        others["unet_A_step"] = unet_step_bench(stream)
        others["unet_T"] = unet_bench(stream, channels=(32, 64, 128, 256, 512), precision="fp16")
    cpu = None if args.no_cpu else cpu_baseline(env)

    line = {
        "metric": METRIC, "value": round(M / (ms * 1e-3), 1), "unit": "voxels/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8" if cfg.precision == "int8" else "fp16", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.H}x{cfg.W} {cfg.precision} refiner step K=1, C={C}, "
                               f"{2 * cfg.n_blocks} conv layers, fit iters {cfg.fit_iters}",
                   "voxels": M, "parallelism": "1 GPU"},
        "final_fit_ms": round(ms_with_final - ms, 5), "step_with_final_fit_ms": round(ms_with_final, 5),
        "wall_s_timed": round(wall, 3),
        "roofline": roofline, "measured_peaks": peaks, "cpu_baseline": cpu, "conv_microbench": micro,
        "other_configs": others,
        "kernel_ms": {k: round(v, 5) for k, v in kern.items()},
        "per_step_ms": {k: round(v, 5) for k, v in per_step.items()},
        "kernel_gbs_contract": {k: round(contract[k] / (kern[k] * 1e-3) / 1e9, 1) for k in kern},
        "kernel_gbs_minimal": {k: round(minimal[k] / (kern[k] * 1e-3) / 1e9, 1) for k in kern},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
