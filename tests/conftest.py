import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# The property tests draw the same examples on every run, so that a run of the suite is
# repeatable; broader searches run the same strategies with more examples outside the suite.
# Loaded before the test modules are imported: their @settings inherit it.
from hypothesis import settings as _hypothesis_settings  # noqa: E402

_hypothesis_settings.register_profile("repeatable", derandomize=True, database=None)
_hypothesis_settings.load_profile("repeatable")


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
