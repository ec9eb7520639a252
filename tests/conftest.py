import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the gfx950 HIP kernels)")


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    # GPU tests fail (never skip) without a GPU: a skipped parity test on a
    # machine meant to run them would hide a broken kernel.
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda", 0)
