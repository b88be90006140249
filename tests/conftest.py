import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on the device)")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from promptmoge_amd import _lib

    _lib.lib()  # must load: GPU tests never fall back
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    """Names the case on stdout before a GPU step, flushed, so a run that dies still says what it was doing."""
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="session")
def libpmg():
    """The built library (built here if missing); loading it needs no GPU."""
    from promptmoge_amd import _lib

    if not _lib.LIB_PATH.exists():
        from promptmoge_amd import build

        build.build()
    return _lib.lib()
