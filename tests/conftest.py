import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from elasticmegatron_amd import _native

    _native.load()  # the native path must be present: no fallback
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _free_device_memory(request):
    """Before each GPU test, free what earlier tests left: full-size states are hundreds of GB."""
    if "gpu_device" in request.fixturenames:
        import gc

        import torch

        gc.collect()
        if torch.cuda.is_available():
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
    yield
