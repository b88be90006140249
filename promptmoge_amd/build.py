"""Builds libpmg.so, the gfx950 HIP library behind promptmoge_amd, in-tree with hipcc.

    python -m promptmoge_amd.build          # or promptmoge_amd.build.build()

Every translation unit is compiled with
  -ffp-contract=off                              no fused multiply-add is formed, so every fp32 operation is
                                                 individually rounded (bit-reproducible against the host and the
                                                 NumPy restatement);
  -fhip-fp32-correctly-rounded-divide-sqrt       IEEE division and square root in device code;
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 instructions are generated.
With PMG_FIT_PHASE_TRACE=1 in the environment the metric fit is compiled with its phase marks (profiling only).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libpmg.so"
SOURCES = ["pmg_api.hip", "pmg_structure.hip", "pmg_conv.hip", "pmg_conv_col.hip", "pmg_rowops.hip", "pmg_fit.hip", "pmg_fill.hip", "pmg_order.hip", "pmg_probe.hip", "pmg_pool.hip", "pmg_gauge.hip", "pmg_unet.hip"]
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    extra = []
    if src == "pmg_fit.hip" and os.environ.get("PMG_FIT_PHASE_TRACE") == "1":
        extra = ["-DPMG_FIT_PHASE_TRACE"]  # the metric fit records its per-round phases (profiling builds only)
    cmd = [_hipcc(), *FLAGS, *extra, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs: int | None = None) -> Path:
    """Compiles every source and links libpmg.so (always rebuilds)."""
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
    sys.exit(0)
