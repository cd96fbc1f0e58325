import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(autouse=True)
def _seed():
    # reference convention: tests/conftest.py:44
    np.random.seed(42)


def gpu_present() -> bool:
    from nkipy_amd.runtime.utils import is_gpu_available

    return is_gpu_available()


@pytest.fixture(scope="session")
def gpu():
    """The process-wide HIP runtime; skips when no GPU is visible."""
    if not gpu_present():
        pytest.skip("no GPU visible")
    from nkipy_amd.runtime.hip import get_runtime

    return get_runtime()
