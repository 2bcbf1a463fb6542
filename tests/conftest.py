import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")
    _build_oracle_generator()


def _build_oracle_generator():
    """The oracle's C generator (oracle/Makefile), built when missing and a compiler is here.

    The oracle falls back to its numpy generator without it, so a failed build is not an error.
    """
    import shutil
    import subprocess

    lib = os.path.join(ROOT, "oracle", "build", "libsynth_ref.so")
    if os.path.exists(lib) or not (shutil.which("make") and shutil.which("gcc")):
        return
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=False,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)


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
