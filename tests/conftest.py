import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "laya-cuda_amd"))
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built liblaya_hip.so")


def gpu_available():
    try:
        import torch
    except ImportError:
        return False
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    """Skip on machines without a GPU; fail loudly if the native library is missing."""
    if not gpu_available():
        pytest.skip("no GPU")
    from laya_cuda import _lib
    _lib.load()
    import torch
    return torch.device("cuda:0")
