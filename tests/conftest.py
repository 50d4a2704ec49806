import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "fast-qr_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import fastqr

    if not fastqr.is_built():
        raise RuntimeError("libfastqr is not built: the GPU tests refuse to run without the native library")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _threads():
    import torch

    torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))
    yield
