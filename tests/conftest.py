import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
if str(ROOT / "tests") not in sys.path:
    sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running test")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip when no GPU is visible; otherwise return the torch device."""
    if not _has_gpu():
        pytest.skip("no GPU visible")
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def w8a8():
    import optimized_rocwmma_samples_amd as w
    w.library()  # raises if libw8a8.so was not built: no fallback
    return w


@pytest.fixture(scope="session")
def orc():
    import oracle_lib
    oracle_lib.oracle()
    return oracle_lib
