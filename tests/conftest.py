import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


def gpu_available() -> bool:
    return torch.cuda.is_available()


requires_gpu = pytest.mark.skipif(not gpu_available(), reason="needs a GPU")


@pytest.fixture(scope="session")
def hip_lib():
    """The built libmykfa.so (GPU tests fail loudly if it is missing: no fallback)."""
    from myk_llm_amd import _lib

    return _lib.lib()


def pytest_report_header(config):
    lines = [f"torch {torch.__version__} hip {torch.version.hip}"]
    if torch.cuda.is_available():
        lines.append(f"device {torch.cuda.get_device_name(0)}")
    return lines


os.environ.setdefault("PYTHONHASHSEED", "0")
