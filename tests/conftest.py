import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


@pytest.fixture(scope="session")
def pe():
    """The product package (prism-engine_amd)."""
    return importlib.import_module("prism-engine_amd")


@pytest.fixture(scope="session")
def oracle():
    """The CPU oracle (test infrastructure)."""
    mod = importlib.import_module("oracle")
    mod.lib()
    return mod


def _gpu_present() -> bool:
    try:
        import torch
        return torch.cuda.is_available() and torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu_ctx(pe):
    """A prism_hip context on device 0.  Skips only when no GPU is present;
    with a GPU, a missing or broken library fails the test."""
    if not _gpu_present():
        pytest.skip("no GPU")
    ctx = pe.Context(0)
    yield ctx
    ctx.close()
