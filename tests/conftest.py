import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import oracle as O
    if not O.LIB_PATH.exists():
        O.build(ref=False)
    return O


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm GPU is visible")
    from joule_amd import _lib
    _lib.lib()  # raises if libjoule_amd.so is missing: no silent fallback
    return torch.device("cuda:0")


def banner(msg: str) -> None:
    """Name the case on stdout before a GPU step, flushed."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()
    os.sync() if hasattr(os, "sync") else None
