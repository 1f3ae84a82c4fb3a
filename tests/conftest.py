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


HALF_ULP_EXP = {"bf16": 8, "f16": 11}  # half an ulp of |y| is 2^(floor(log2|y|) - this)


def half_ulp(values, dtype):
    """Half a unit in the last place of `dtype` at each value (0 for f32): the
    largest error the final store of a correctly computed result may add."""
    import numpy as np

    if dtype not in HALF_ULP_EXP:
        return np.zeros(np.shape(values))
    v = np.abs(np.asarray(values, dtype=np.float64))
    e = np.floor(np.log2(np.where(v > 0, v, 1.0)))
    return np.where(v > 0, np.ldexp(1.0, (e - HALF_ULP_EXP[dtype]).astype(np.int64)), 0.0)


def assert_out(actual, expected, eps, out_dtype, what="", half_ulps=1):
    """Parity bar for a kernel output stored as `out_dtype`:
    |a - e| <= eps + eps*max(|a|,|e|) + half_ulps * half_ulp(out_dtype, max(|a|,|e|)).
    eps (2e-3 for bf16/f16 inputs, 1e-5 for f32) bounds the fp32 arithmetic;
    the half ulp is the output store's own rounding (bf16 alone can round by
    2^-8 relative, above 2e-3). An intermediate the reference stores and then
    re-reads may sit one rounding step away (half_ulps=2)."""
    import numpy as np

    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    m = np.maximum(np.abs(a), np.abs(e))
    ok = np.abs(a - e) <= eps + eps * m + half_ulps * half_ulp(m, out_dtype)
    if not np.all(ok):
        bad = np.flatnonzero(~ok.ravel())
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size}/{ok.size} elements outside eps={eps} (+half ulp {out_dtype}); first at {i}: "
            f"{a.ravel()[i]!r} vs {e.ravel()[i]!r}; max|d|={np.nanmax(np.abs(a - e)):.3e}"
        )


@pytest.fixture(scope="session")
def oracle():
    import oracle as O

    O.lib()
    return O
