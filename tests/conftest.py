import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(autouse=True)
def _seed():
    # reference convention: tests/conftest.py:44
    np.random.seed(42)


def gpu_present() -> bool:
    from nkipy_amd.runtime.utils import is_gpu_available

    return is_gpu_available()


@pytest.fixture
def gpu():
    """The process-wide HIP runtime (re-read per test, since a test may reset
    it); skips when no GPU is visible."""
    if not gpu_present():
        pytest.skip("no GPU visible")
    from nkipy_amd.runtime.hip import get_runtime

    return get_runtime()


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Print the achieved parity errors of every check that ran."""
    try:
        from parity import RECORDS
    except ImportError:
        return
    if not RECORDS:
        return
    tr = terminalreporter
    tr.section("achieved parity errors")
    for r in RECORDS:
        tr.write_line(f"{r['check']:<58} n={r['n']:<10} max_abs={r['max_abs']:.3e} "
                      f"max_rel={r['max_rel']:.3e} worst/bar={r['worst_of_bar']:.3f}"
                      + (f" rounding-step flips={r['flips']}" if r.get("flips") else ""))
