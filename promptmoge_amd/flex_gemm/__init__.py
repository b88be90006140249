"""A `flex_gemm` package on libpmg.so for PromptMoGe's plug point (promptmoge/model.py:29-30 only falls back to its
bundled pure-PyTorch flex_gemm when no `flex_gemm` is importable).

    import promptmoge_amd.flex_gemm as fg
    fg.install()          # registers this package as `flex_gemm` (and `flex_gemm.nn`, `flex_gemm.ops`)
    # then: from flex_gemm.nn import SubmanifoldConv3d; from flex_gemm.ops import NeighborCache
"""
from __future__ import annotations

import sys

from . import nn, ops

__all__ = ["nn", "ops", "install"]


def install() -> None:
    """Makes `import flex_gemm` (and importlib.util.find_spec("flex_gemm")) resolve to this package."""
    pkg = sys.modules[__name__]
    sys.modules["flex_gemm"] = pkg
    sys.modules["flex_gemm.nn"] = nn
    sys.modules["flex_gemm.ops"] = ops
