import importlib
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs on the GPU box)")


@pytest.fixture(scope="session")
def pkg():
    return importlib.import_module("safetyraise-lmengine_amd")


@pytest.fixture(scope="session")
def backend(pkg):
    """Plugin loaded the way the engine loads it; GPU tests only."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a GPU")
    torch.cuda.init()
    b = pkg.NativeBackend.load()
    yield b
    b.close()
