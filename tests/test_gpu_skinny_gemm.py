"""GPU parity of the skinny Matmul (2 <= M <= 64, transposeB, f16 and bf16
with f32 accumulation; the role of the reference's small-M MPP tiles,
Matmul.swift:175-196, MPPMatmul.metal:19-91) against the oracle's Matmul
loop (KernelsTests.swift:239-267 order)."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_out
from gpu_util import EPS, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _gemm(env, a, b, at, ot, guard=0):
    """C = a . b^T through Kernels.Matmul; with `guard` elements of NaN past
    C's end, which must stay untouched."""
    pa, lib, stream, enc = env
    M, K = a.shape
    N = b.shape[0]
    buf = upload(pa, np.full(M * N + guard, np.nan, np.float32), ot)
    c = buf.view([M, N])
    k = pa.Kernels.Matmul(upload(pa, a, at), upload(pa, b, at), c, True)
    enc.encode(k)
    stream.synchronize()
    out = download(buf, stream)
    if guard:
        assert np.isnan(out[M * N:]).all(), "the skinny GEMM wrote past C"
    return out[:M * N].reshape(M, N), k


@pytest.mark.parametrize("at,ot", [("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("M,K,N", [(2, 64, 67), (8, 2304, 9216), (8, 2304, 2304), (16, 136, 300), (17, 520, 129),
                                   (33, 256, 1000), (48, 2048, 64), (64, 3072, 512), (5, 8, 33), (63, 40, 31)])
def test_skinny_matmul_vs_oracle(env, at, ot, M, K, N):
    a = rounded(O.normal(M * 7 + K, (M, K)), at)
    b = rounded(O.normal(N * 3 + K, (N, K), std=0.02), at)
    got, k = _gemm(env, a, b, at, ot, guard=64)
    assert k.function_names == [f"matmul_skinny_{at}_{at}_{ot}_m{16 * (-(-M // 16))}"]
    ref = O.matmul(a, b, M, K, N, True).reshape(M, N)
    # inputs exact in their dtype, f32 accumulation in another order: 1e-5
    # for f32 outputs, else the 16-bit bar plus the store's rounding
    assert_out(got, ref, 1e-5 if ot == "f32" else EPS[at], ot, f"skinny gemm {at}->{ot} {M}x{K}x{N}")


@pytest.mark.parametrize("at", ["f16", "bf16"])
@pytest.mark.parametrize("M,K,N", [(3, 320, 160), (16, 1000, 64), (40, 96, 250), (64, 4104, 96)])
def test_skinny_matmul_integer_exact(env, at, M, K, N):
    # small integers: every product and partial sum is exact in f32, so the
    # result is exact whatever the order (K-split over waves, LDS sum): pins
    # every fragment index, the row clamps and the K tail
    rng = np.random.default_rng(M * 1000 + K)
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (N, K)).astype(np.float32)
    got, _ = _gemm(env, a, b, at, "f32", guard=16)
    np.testing.assert_array_equal(got, (a.astype(np.int64) @ b.T.astype(np.int64)).astype(np.float32))
