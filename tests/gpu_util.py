"""Helpers for the GPU parity tests: upload/download through the C ABI with the
oracle's conversions, and the tolerances the parity bar states."""
import numpy as np
import pytest

import oracle as O

TAG = {"f32": O.F32, "f16": O.F16, "bf16": O.BF16}
# north_star bar: f32 within 1e-5, f16/bf16 within 2e-3 (fp32 accumulation),
# in the reference's approxEqual form |a-b| <= eps + eps*max(|a|,|b|)
EPS = {"f32": 1e-5, "f16": 2e-3, "bf16": 2e-3}


def gpu_env():
    import popcorn_amd as pa

    if pa.device_count() < 1:
        pytest.skip("no GPU visible")
    lib = pa.KernelLibrary()
    stream = pa.Stream()
    enc = pa.KernelCommandEncoder(lib, stream)
    return pa, lib, stream, enc


def rounded(x, dtype):
    """f32 values after a store in `dtype` (what a tensor of that dtype holds)."""
    return O.round_to(np.asarray(x, np.float32), TAG[dtype])


def upload(pa, values, dtype, stream=None):
    values = np.asarray(values, np.float32)
    if dtype == "f32":
        return pa.Tensor.from_numpy(values, "f32", stream)
    return pa.Tensor.from_numpy(O.to_bits(values, TAG[dtype]), dtype, stream)


def download(t, stream=None):
    raw = t.numpy(stream)
    if t.dtype == "f32":
        return raw
    if t.dtype in ("bf16", "f16"):
        return O.from_bits(raw.view(np.uint16), TAG[t.dtype])
    return raw
