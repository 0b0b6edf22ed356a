import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible HIP device")
    from kunserve_amd import _lib

    _lib.lib()  # raises if the library was not built
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _release_gpu_memory(request):
    yield
    if request.node.get_closest_marker("gpu"):
        import torch

        if torch.cuda.is_available():
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
