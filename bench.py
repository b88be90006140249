#!/usr/bin/env python3
"""Benchmark of the MI355X refiner step (one JSON line on stdout).

Workload (the headline): a Model-A-shape (480x640) int8 refiner step, K=1: prompt fit
(trimmed LS, 10 trim rounds) -> prompt residual/gate -> voxelise (M = 307,200 voxels) -> column neighbour map ->
input_proj + prompt_proj -> 3 residual blocks = 6 int8 submanifold 3x3x3 conv layers at C=48 -> out_proj -> logz +=
delta, on synthetic seeded inputs (promptmoge_amd.spec) already resident in HBM. One "step" is one replay of the
captured HIP graph of that chain; the metric fit of the refined depth is timed separately (`final_fit_ms`).

    value   active voxels refined per second = M / step time (whole job; one GPU)
    roofline  the dominant kernel of the step (largest time per step), algorithmic bytes per launch / its average
              duration, both measured here with HIP events on the stream it runs on (standalone launches of the
              step's own kernels on the step's data)
    cpu_baseline  the oracle's restatement of the reference's CPU path (_fallback conv on fake-quantised operands,
              fit_scale_shift with an exact k-th selection) timed on this host on one Model-A step
    conv_microbench  isolated int8 conv on 1,000,000 surface voxels in 1024^3, C = 64 and 128
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
METRIC = "refiner step latency ms + active voxels/s at 480×640; int8 conv TOPS (% peak)"


def _events_ms(fn, reps, stream):
    import torch

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="A", choices=["A", "B", "T", "H"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-micro", action="store_true", help="skip the 1M-voxel conv microbench")
    ap.add_argument("--kernel-reps", type=int, default=50)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the refiner step is per frame and this build uses no collectives); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from promptmoge_amd import ops, spec
    from promptmoge_amd.refiner import RefinerStep

    dev = torch.device("cuda:0")
    cfg = spec.CONFIGS[args.config]
    sc = spec.make_scene(cfg)
    w = spec.refiner_for(cfg, sc)
    M, C = cfg.M, cfg.C
    stream = torch.cuda.Stream()
    out = {}
    with torch.cuda.stream(stream):
        P = torch.from_numpy(sc.points[None].copy()).to(dev)
        Pout = torch.empty_like(P)
        L = torch.from_numpy(sc.lidar[None].copy()).to(dev)
        Cf = torch.from_numpy(sc.conf[None].copy()).to(dev)
        step = RefinerStep(w, 1, cfg.H, cfg.W, precision=cfg.precision, fit_iters=cfg.fit_iters)
        for _ in range(args.warmup):
            step(P, L, Cf, out=Pout)
        step.check()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ms = _events_ms(lambda: step(P, L, Cf, out=Pout), args.steps, stream)
        wall = time.perf_counter() - t0
        step.check()

        stepf = RefinerStep(w, 1, cfg.H, cfg.W, precision=cfg.precision, fit_iters=cfg.fit_iters, final_fit=True)
        for _ in range(5):
            stepf(P, L, Cf, out=Pout)
        ms_with_final = _events_ms(lambda: stepf(P, L, Cf, out=Pout), 50, stream)
        stepf.check()

        # ---- per-kernel timing with the step's own shapes and data (standalone launches of the step's kernels)
        reps = args.kernel_reps
        zq, _, _ = ops.voxelize(P[..., 2:], 256.0, stride=3, shape=(1, cfg.H, cfg.W))
        x = step.buffer("x")
        b0, b1 = step.weights.blocks[0], step.weights.blocks[-1]
        q1 = ops.ln_silu_quant(x, b0["gamma"], b0["beta"], b0["m1"])
        q2 = ops.spconv_col(q1, zq, b0["w1"], ops.EPI_Q, a_scale=b0["a1"], w_scale=b0["s1"], bias=b0["b1"],
                            out_mult=b0["m2"])
        xr = x.clone()
        nq = torch.empty_like(q1)
        kern = {}
        kern["fit_prompt"] = _events_ms(lambda: ops.fit_prompt(P, L, Cf, iters=cfg.fit_iters), reps, stream)
        kern["conv_q"] = _events_ms(lambda: ops.spconv_col(q1, zq, b0["w1"], ops.EPI_Q, a_scale=b0["a1"],
                                                           w_scale=b0["s1"], bias=b0["b1"], out_mult=b0["m2"],
                                                           out=q2), reps, stream)
        kern["conv_rln"] = _events_ms(lambda: ops.spconv_col(q2, zq, b0["w2"], ops.EPI_RLN, a_scale=b0["a2"],
                                                             w_scale=b0["s2"], bias=b0["b2"], skip=xr, out=xr,
                                                             ln_gamma=b1["gamma"], ln_beta=b1["beta"],
                                                             next_mult=b1["m1"], next_q=nq), reps, stream)
        kern["conv_rout"] = _events_ms(lambda: ops.spconv_col(q2, zq, b1["w2"], ops.EPI_ROUT, a_scale=b1["a2"],
                                                              w_scale=b1["s2"], bias=b1["b2"], skip=x,
                                                              out_w=step.weights.out_w, out_b=step.weights.out_b,
                                                              points=P, points_out=Pout), reps, stream)
        nb = cfg.n_blocks
        per_step = {"fit_prompt": kern["fit_prompt"], "conv_q": nb * kern["conv_q"],
                    "conv_rln": (nb - 1) * kern["conv_rln"], "conv_rout": kern["conv_rout"]}
        per_step["input_stage_and_launch_gaps"] = max(ms - sum(per_step.values()), 0.0)
        dominant = max((k for k in per_step if k in kern), key=per_step.get)
        # algorithmic bytes per launch (every byte the kernel must move at least once)
        wb = 27 * C * C
        alg = {
            "fit_prompt": M * 12,                           # logz, LiDAR, conf: 4 B each
            "conv_q": M * (C + 4 + C) + wb,                 # codes in, keys, codes out, weights
            "conv_rln": M * (C + 4 + 4 * C + 4 * C + C) + wb,  # codes, keys, residual in/out, next codes
            "conv_rout": M * (C + 4 + 4 * C + 12 + 12) + wb,  # codes, keys, residual, point map in/out
        }
        ach = alg[dominant] / (kern[dominant] * 1e-3) / 1e9
        out["breakdown_ms"] = {k: round(v, 5) for k, v in kern.items()}
        out["per_step_ms_est"] = {k: round(v, 5) for k, v in per_step.items()}
        out["kernel_gbs"] = {k: round(alg[k] / (kern[k] * 1e-3) / 1e9, 1) for k in kern}
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                    "algorithmic_bytes": int(alg[dominant]), "avg_launch_ms": round(kern[dominant], 5)}

    # ---- conv microbench
    micro = None
    if not args.no_micro:
        coords = spec.make_voxels(1_000_000, 1024, seed=21)
        with torch.cuda.stream(stream):
            cd = torch.from_numpy(coords).to(dev)
            shape = (1, 1024, 1024, 1024)
            ntu, tmu, _ = ops.nmap_hash(cd, shape)
            torch.cuda.synchronize()
            hash_ms = _events_ms(lambda: ops.nmap_hash(cd, shape), 10, stream)
            pu = int((ntu >= 0).sum().item())
            micro = {"voxels": int(coords.shape[0]), "pairs": pu, "mean_active_taps": round(pu / coords.shape[0], 3),
                     "hash_map_ms": round(hash_ms, 4)}
            g = torch.Generator(device="cpu").manual_seed(5)
            for Cm in (64, 128):
                xm = torch.randint(-127, 128, (coords.shape[0], Cm), generator=g, dtype=torch.int8).to(dev)
                wm = torch.randint(-127, 128, (Cm, 3, 3, 3, Cm), generator=g, dtype=torch.int8).to(dev)
                sm = torch.full((Cm,), 1e-4, device=dev)
                om = torch.empty((coords.shape[0], Cm), dtype=torch.int8, device=dev)
                f = lambda: ops.spconv_i8(xm, ntu, tmu, wm, ops.EPI_Q, a_scale=0.01, w_scale=sm, out_mult=20.0, out=om)
                f()
                t = _events_ms(f, 10, stream)
                tops = 2 * Cm * Cm * pu / (t * 1e-3) / 1e12
                micro[f"C{Cm}"] = {"ms": round(t, 4), "tops": round(tops, 2), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}

    # ---- CPU baseline: the oracle's restatement of the reference CPU path, one Model-A step
    cpu = None
    if not args.no_cpu:
        from oracle import refiner as orf

        try:
            from threadpoolctl import threadpool_info

            threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
        except Exception:
            threads = os.cpu_count() or 1
        t0 = time.perf_counter()
        orf.step_fakequant(sc.points[None], sc.lidar[None], sc.conf[None], w, iters=cfg.fit_iters)
        tc = time.perf_counter() - t0
        cpu = {"value": round(M / tc, 1), "unit": "voxels/s", "cores": int(threads), "kind": "port",
               "sample": f"1 step of config {cfg.name} ({M} voxels), NumPy (BLAS {threads} threads, elementwise 1)",
               "ms_per_step": round(tc * 1e3, 1)}

    line = {
        "metric": METRIC, "value": round(M / (ms * 1e-3), 1), "unit": "voxels/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8" if cfg.precision == "int8" else "fp16", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.H}x{cfg.W} {cfg.precision} refiner step K=1, C={C}, "
                               f"{2 * cfg.n_blocks} conv layers, fit iters {cfg.fit_iters}",
                   "voxels": M, "parallelism": "1 GPU"},
        "final_fit_ms": round(ms_with_final - ms, 5), "step_with_final_fit_ms": round(ms_with_final, 5),
        "wall_s_timed": round(wall, 3),
        "roofline": roofline, "cpu_baseline": cpu, "conv_microbench": micro, **out,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
