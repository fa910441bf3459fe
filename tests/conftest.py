import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen2-7b-triton_engine_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The CUDA/HIP device for GPU tests; skips only when no GPU is present.

    With a GPU present, a missing HIP library is a failure, not a skip.
    """
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")
