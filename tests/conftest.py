import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C-ABI library")


def approx_equal(a, b, eps):
    """The reference's comparison (Tests/PopcornTests/Kernels/KernelsTests.swift:72-74):
    |a - b| <= eps + eps * max(|a|, |b|), elementwise."""
    import numpy as np

    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.abs(a - b) <= eps + eps * np.maximum(np.abs(a), np.abs(b))


def assert_approx(actual, expected, eps, what=""):
    import numpy as np

    ok = approx_equal(actual, expected, eps)
    if not np.all(ok):
        a = np.asarray(actual, dtype=np.float64).ravel()
        e = np.asarray(expected, dtype=np.float64).ravel()
        bad = np.flatnonzero(~ok.ravel())
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size}/{ok.size} elements outside eps={eps}; first at {i}: "
            f"{a[i]!r} vs {e[i]!r}; max|d|={np.nanmax(np.abs(a - e)):.3e}"
        )


@pytest.fixture(scope="session")
def oracle():
    import oracle as O

    O.lib()
    return O
